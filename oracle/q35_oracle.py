"""ctypes binding of the CPU oracle (q35_oracle.c) and of the reference build
in oracle/_ref. TEST INFRASTRUCTURE ONLY: imported by tests/, by
__graft_entry__.smoke() and by bench.py's cpu_baseline leg as the checker;
never part of the measured or shipped path.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, c_float, c_int, c_int16, c_int32, c_size_t, c_uint16, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_DIR = os.path.join(HERE, "_ref")
REF_SO = os.path.join(REF_DIR, "libq35ref.so")
SIGN_SEED = 0x5148333548313238


def _build_oracle():
    if not os.path.exists(ORACLE_SO):
        subprocess.run(["make", "-C", HERE, "oracle"], check=True, stdout=subprocess.DEVNULL)


_build_oracle()
lib = ctypes.CDLL(ORACLE_SO)

# numpy record layouts of the reference blocks (q4_0.h:36-70)
Q4X8 = np.dtype([("d", "<u2", (8,)), ("qs", "u1", (128,))])
Q8X4 = np.dtype([("scales", "<f4", (4,)), ("sums", "<i2", (4,)), ("qs", "i1", (128,))])
Q8X1 = np.dtype([("scales", "<f4", (1,)), ("sums", "<i2", (1,)), ("qs", "i1", (32,)), ("pad", "<i2")])
Q4_0 = np.dtype([("d", "<u2"), ("qs", "u1", (16,))])
G16 = np.dtype([("d", "<u2", (2, 8)), ("qs", "u1", (128,))])      # q4_g16.h:5-6
Q8_0 = np.dtype([("d", "<u2"), ("qs", "i1", (32,))])                # q4_0.h:13-16
assert Q4X8.itemsize == 144 and Q8X4.itemsize == 152 and Q8X1.itemsize == 40 and Q4_0.itemsize == 18
assert G16.itemsize == 160 and Q8_0.itemsize == 34

P = c_void_p
for name, res, args in [
    ("q35o_float_to_half", c_uint16, [c_float]),
    ("q35o_half_to_float", c_float, [c_uint16]),
    ("q35o_attention_float_to_half", c_uint16, [c_float]),
    ("q35o_attention_store_f16", None, [P, P, c_size_t]),
    ("q35o_q8_quantize_vector_1", None, [P, P, c_size_t]),
    ("q35o_q8_quantize_vectors_4", None, [P, P, c_size_t, c_size_t]),
    ("q35o_h128_sign_word", c_uint64, [c_size_t, c_size_t, c_uint64]),
    ("q35o_h128_transform_unscaled", None, [P, P, c_size_t, c_uint64]),
    ("q35o_h128_transform", None, [P, P, c_size_t, c_uint64]),
    ("q35o_h128_prepare_activation_1", c_int, [P, P, c_size_t, c_uint64]),
    ("q35o_h128_prepare_activations_4", c_int, [P, P, c_size_t, c_size_t, c_uint64]),
    ("q35o_q4_quantize_transformed", None, [P, P, c_size_t]),
    ("q35o_h128_quantize_matrix", c_int, [P, P, c_size_t, c_size_t, c_uint64]),
    ("q35o_dot4_pack_rows_8", None, [P, P, c_size_t, c_size_t]),
    ("q35o_dot4_unpack_rows_8", None, [P, P, c_size_t, c_size_t]),
    ("q35o_dot4_dequantize_row", None, [P, c_size_t, P, c_size_t]),
    ("q35o_dot4_block_dots", None, [P, P, P, P, c_size_t, c_size_t]),
    ("q35o_dot4_matvec", None, [P, P, P, c_size_t, c_size_t]),
    ("q35o_dot4_matmul", None, [P, P, P, c_size_t, c_size_t, c_size_t, c_size_t]),
    ("q35o_dot4_argmax", None, [P, P, P, c_float, c_size_t, c_size_t, c_size_t, P, P]),
    ("q35o_delta_net_update_rows", None, [P, P, P, P, P, P, P, c_size_t, c_size_t, c_size_t, c_size_t]),
    ("q35o_attention_decode", None, [P, P, P, P, P, P, c_size_t, c_int, c_int, c_int, c_int, c_float,
                                     c_size_t, c_size_t]),
    ("q35o_rms_norm", None, [P, P, P, c_size_t, c_size_t, c_float, c_float]),
    ("q35o_l2_normalize", None, [P, c_size_t, c_size_t, c_float, c_float]),
    ("q35o_conv1d_silu", None, [P, c_size_t, P, P, P, c_size_t, c_size_t]),
    ("q35o_silu_mul", None, [P, P, P, c_size_t]),
    ("q35o_rope", None, [P, c_size_t, c_size_t, c_size_t, P, P]),
    ("q35o_sigmoid", c_float, [c_float]),
    ("q35o_softplus", c_float, [c_float]),
    ("q35o_rope_tables", None, [c_float, c_int, c_size_t, P, P]),
    ("q35o_g16_dequantize_row", None, [P, c_size_t, P, c_size_t]),
    ("q35o_g16_matmul", None, [P, P, P, c_size_t, c_size_t, c_size_t, c_size_t]),
    ("q35o_q8_matmul", None, [P, P, P, P, c_size_t, c_size_t, c_size_t, c_size_t]),
]:
    f = getattr(lib, name)
    f.restype, f.argtypes = res, args


def ptr(a):
    return c_void_p(a.ctypes.data) if a is not None else None


# ------------------------------------------------------------ kernel helpers

def random_q4_blocks(rng, rows, cols, scales=None):
    """Canonical Q4_0 blocks [rows, cols/32]: codes U{0..15}, FP16 scales lognormal(0, 0.5)."""
    b = np.zeros((rows, cols // 32), Q4_0)
    b["qs"] = rng.integers(0, 256, size=(rows, cols // 32, 16), dtype=np.uint8)
    if scales is None:
        scales = rng.lognormal(0.0, 0.5, size=(rows, cols // 32)).astype(np.float16)
    b["d"] = np.asarray(scales, np.float16).view(np.uint16)
    return b


def dot4_pack(canon, rows, blocks):
    out = np.zeros((rows // 8, blocks), Q4X8)
    lib.q35o_dot4_pack_rows_8(ptr(canon), ptr(out), rows, blocks)
    return out


def dot4_unpack(packed, rows, blocks):
    out = np.zeros((rows, blocks), Q4_0)
    lib.q35o_dot4_unpack_rows_8(ptr(packed), ptr(out), rows, blocks)
    return out


def q8_quantize_1(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.size // 32, Q8X1)
    lib.q35o_q8_quantize_vector_1(ptr(x), ptr(out), x.size // 32)
    return out


def q8_quantize_4(x):
    x = np.ascontiguousarray(x, np.float32)
    v, cols = x.shape
    out = np.zeros((v // 4, cols // 32), Q8X4)
    lib.q35o_q8_quantize_vectors_4(ptr(x), ptr(out), v, cols // 32)
    return out


def h128_prepare_1(x, seed=SIGN_SEED):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.size // 32, Q8X1)
    assert lib.q35o_h128_prepare_activation_1(ptr(x), ptr(out), x.size, seed) == 1
    return out


def h128_prepare_4(x, seed=SIGN_SEED):
    x = np.ascontiguousarray(x, np.float32)
    v, cols = x.shape
    out = np.zeros((v // 4, cols // 32), Q8X4)
    assert lib.q35o_h128_prepare_activations_4(ptr(x), ptr(out), v, cols, seed) == 1
    return out


def h128_transform(x, block=0, seed=SIGN_SEED, scaled=True):
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(128, np.float32)
    (lib.q35o_h128_transform if scaled else lib.q35o_h128_transform_unscaled)(ptr(x), ptr(y), block, seed)
    return y


def h128_quantize_matrix(w, seed=SIGN_SEED):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    out = np.zeros((rows, cols // 32), Q4_0)
    assert lib.q35o_h128_quantize_matrix(ptr(w), ptr(out), rows, cols, seed) == 1
    return out


def q4_quantize(w):
    """Identity-basis Q4 (absmax/7) blocks of a [rows, cols] matrix."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    out = np.zeros((rows, cols // 32), Q4_0)
    lib.q35o_q4_quantize_transformed(ptr(w), ptr(out), rows * cols // 32)
    return out


def g16_pack(w):
    """Fixture packer for Q4G16Tile [rows/8, cols/32] (q4_g16.h:5-6): per row,
    block and 16-column half an absmax/7 binary16 scale and codes
    round(x / d) + 8 clamped to 0..15, in the DOT4 nibble order
    (q4_g16.cpp:31-34). Any such tile is a valid G16 input; the reference's
    MSE16 quantizer only chooses scales differently."""
    w = np.asarray(w, np.float32)
    rows, cols = w.shape
    nb = cols // 32
    x = w.reshape(rows, nb, 2, 16)
    d = (np.abs(x).max(axis=3) / 7.0).astype(np.float16)
    df = d.astype(np.float32)
    inv = np.where(df > 0, 1.0 / np.where(df > 0, df, 1), 0.0).astype(np.float32)
    q = (np.clip(np.round(x * inv[..., None]), -8, 7) + 8).astype(np.uint8).reshape(rows, nb, 32)
    out = np.zeros((rows // 8, nb), G16)
    dd = d.view(np.uint16).reshape(rows // 8, 8, nb, 2)
    out["d"] = dd.transpose(0, 2, 3, 1)
    i = np.arange(32)
    byte = 32 * (i // 8) + (i % 4)   # + 4 * row
    shift = np.where(i % 8 < 4, 0, 4)
    qs = np.zeros((rows // 8, nb, 128), np.uint16)
    qr = q.reshape(rows // 8, 8, nb, 32)
    for r in range(8):
        for k in range(32):
            qs[:, :, byte[k] + 4 * r] |= (qr[:, r, :, k].astype(np.uint16) << np.uint16(shift[k])).astype(np.uint16)
    out["qs"] = qs.astype(np.uint8)
    return out


def g16_dequantize_row(tiles, row, blocks):
    out = np.zeros(blocks * 32, np.float32)
    lib.q35o_g16_dequantize_row(ptr(tiles), row, ptr(out), blocks)
    return out


def g16_matmul(tiles, act1, rows, count, blocks, stride=None):
    """act1: X1 blocks [count * blocks] -> float32 [count, stride]."""
    stride = stride or rows
    out = np.zeros((count, stride), np.float32)
    lib.q35o_g16_matmul(ptr(tiles), ptr(act1), ptr(out), rows, count, blocks, stride)
    return out


def q8_rows_pack(w):
    """Row-major Q8_0 blocks [rows, cols/32] (q8_0_quantize, q8_0.cpp:86-110,
    the same rounding as q8_0_quantize_vector_1) and their F32 scales
    (q8_0_scales_to_f32, as the loader keeps them, weights.inl:741-742)."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    x1 = q8_quantize_1(w.reshape(-1)).reshape(rows, cols // 32)
    out = np.zeros((rows, cols // 32), Q8_0)
    out["qs"] = x1["qs"]
    out["d"] = x1["scales"][..., 0].astype(np.float16).view(np.uint16)
    return out, np.ascontiguousarray(x1["scales"][..., 0], np.float32)


def q8_matmul(blocks8, mscales, act1, rows, count, blocks, stride=None):
    stride = stride or rows
    out = np.zeros((count, stride), np.float32)
    lib.q35o_q8_matmul(ptr(blocks8), ptr(mscales), ptr(act1), ptr(out), rows, count, blocks, stride)
    return out


def silu_mul(gate, up):
    """silu_mul_f32 (activation.cpp:329-357) over matching FP32 vectors."""
    gate = np.ascontiguousarray(gate, np.float32)
    up = np.ascontiguousarray(up, np.float32)
    out = np.zeros_like(gate)
    lib.q35o_silu_mul(ptr(gate), ptr(up), ptr(out), gate.size)
    return out


def rms_norm(x, w, eps, offset):
    """rms_norm_f32 (activation.cpp:224-262) over the rows of x [rows][width]."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    rows, width = x.reshape(-1, x.shape[-1]).shape
    out = np.zeros_like(x)
    lib.q35o_rms_norm(ptr(x), ptr(w), ptr(out), rows, width, eps, offset)
    return out


def dot4_matvec(packed, act1, rows, blocks):
    out = np.zeros(rows, np.float32)
    lib.q35o_dot4_matvec(ptr(packed), ptr(act1), ptr(out), rows, blocks)
    return out


def dot4_matmul(packed, act4, rows, count, blocks, stride=None):
    stride = stride or rows
    out = np.zeros((count, stride), np.float32)
    lib.q35o_dot4_matmul(ptr(packed), ptr(act4), ptr(out), rows, count, blocks, stride)
    return out


def dot4_block_dots(packed, codes, rows, blocks):
    """codes: int8 [blocks*32] of one vector -> int32 [rows, blocks]."""
    codes = np.ascontiguousarray(codes, np.int8)
    out = np.zeros((rows, blocks), np.int32)
    lib.q35o_dot4_block_dots(ptr(packed), ptr(codes), None, ptr(out), rows, blocks)
    return out


def dot4_dequantize_row(packed, row, blocks):
    out = np.zeros(blocks * 32, np.float32)
    lib.q35o_dot4_dequantize_row(ptr(packed), row, ptr(out), blocks)
    return out


def x4_vector(act4, t):
    """Codes, scales and sums of token t from X4 blocks [tiles, blocks]."""
    tile = act4[t // 4]
    return (tile["qs"][:, (t % 4) * 32:(t % 4) * 32 + 32].reshape(-1), tile["scales"][:, t % 4].copy(),
            tile["sums"][:, t % 4].copy())


def delta_rows(state, q, k, v, alpha, beta, kdim, vdim, begin=None, end=None):
    state = np.ascontiguousarray(state, np.float32).copy()
    heads = alpha.size
    out = np.zeros(heads * vdim, np.float32)
    begin = 0 if begin is None else begin
    end = heads * vdim if end is None else end
    lib.q35o_delta_net_update_rows(ptr(state), ptr(np.ascontiguousarray(q, np.float32)),
                                   ptr(np.ascontiguousarray(k, np.float32)),
                                   ptr(np.ascontiguousarray(v, np.float32)),
                                   ptr(np.ascontiguousarray(alpha, np.float32)),
                                   ptr(np.ascontiguousarray(beta, np.float32)), ptr(out), kdim, vdim, begin, end)
    return state, out


def attention_decode(q, gates, keys, values, heads, kv_heads, head_dim, scale=None):
    """q, gates [heads*head_dim]; keys/values FP16 bits [seq, kv_heads*head_dim]."""
    seq = keys.shape[0]
    scale = 1.0 / np.sqrt(head_dim) if scale is None else scale
    keys = np.ascontiguousarray(keys, np.uint16)
    values = np.ascontiguousarray(values, np.uint16)
    krow = (c_void_p * seq)(*[keys.ctypes.data + i * keys.strides[0] for i in range(seq)])
    vrow = (c_void_p * seq)(*[values.ctypes.data + i * values.strides[0] for i in range(seq)])
    scores = np.zeros(heads * seq, np.float32)
    out = np.zeros(heads * head_dim, np.float32)
    lib.q35o_attention_decode(ptr(np.ascontiguousarray(q, np.float32)), ptr(np.ascontiguousarray(gates, np.float32)),
                              ctypes.cast(krow, c_void_p), ctypes.cast(vrow, c_void_p), ptr(scores), ptr(out),
                              heads * head_dim, seq, heads, kv_heads, head_dim, float(scale), 0, heads)
    return out


def f16_bits(x):
    """attention_cache_store_f16's binary16 bits of every value."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.shape, np.uint16)
    lib.q35o_attention_store_f16(ptr(x), ptr(out), x.size)
    return out


def rope_tables(theta, rope_dim, positions):
    """CpuEngine's RoPE tables (cpu_engine.inl:339-352): cosine, sine [positions][rope_dim / 2]."""
    half = rope_dim // 2
    cs = np.zeros((positions, half), np.float32)
    sn = np.zeros((positions, half), np.float32)
    lib.q35o_rope_tables(c_float(theta), rope_dim, positions, ptr(cs), ptr(sn))
    return cs, sn


# ------------------------------------------------------------- whole model

class Dims(ctypes.Structure):
    _fields_ = [("n_layers", c_int), ("hidden", c_int), ("intermediate", c_int), ("vocab", c_int),
                ("n_heads", c_int), ("n_kv_heads", c_int), ("head_dim", c_int), ("rope_dim", c_int),
                ("rope_theta", c_float), ("rms_eps", c_float),
                ("lin_kernel", c_int), ("lin_k_heads", c_int), ("lin_v_heads", c_int),
                ("lin_k_dim", c_int), ("lin_v_dim", c_int), ("sign_seed", c_uint64)]


class Layer(ctypes.Structure):
    _fields_ = [("is_linear", c_int), ("in_proj", P), ("out_proj", P), ("gate_up", P), ("down", P),
                ("input_norm", P), ("post_norm", P), ("conv_w", P), ("lin_norm", P), ("a_log", P),
                ("dt_bias", P), ("q_norm", P), ("k_norm", P), ("gate_rows", c_int), ("gate_q8", P),
                ("gate_scales", P)]


class Weights(ctypes.Structure):
    _fields_ = [("embed", P), ("embed_g16", P), ("final_norm", P), ("layers", POINTER(Layer))]


class State(ctypes.Structure):
    _fields_ = [("conv_state", POINTER(P)), ("conv_ring", POINTER(c_size_t)), ("recurrent", POINTER(P)),
                ("keys", POINTER(P)), ("values", POINTER(P)), ("counts", POINTER(c_int)),
                ("position", c_size_t), ("capacity", c_size_t)]


lib.q35o_linear_attention_row.restype = c_int
lib.q35o_linear_attention_row.argtypes = [POINTER(Dims), POINTER(Layer), P, POINTER(c_size_t), P, P, P]
lib.q35o_full_attention_row.restype = c_int
lib.q35o_full_attention_row.argtypes = [POINTER(Dims), POINTER(Layer), P, P, c_size_t, P, P, P, P]
lib.q35o_forward_batch.restype = c_int
lib.q35o_forward_batch.argtypes = [POINTER(Dims), POINTER(Weights), POINTER(POINTER(State)), P, c_size_t,
                                   c_float, P, P, P]


def dims_from(d):
    """Oracle Dims from any object with the RuntimeDims field names."""
    o = Dims()
    for f, _ in Dims._fields_:
        setattr(o, f, getattr(d, f) if not isinstance(d, dict) else d[f])
    return o


class OracleModel:
    """Weights given as {hf_name: (encoding, shape, payload ndarray)} (artifact naming)."""

    def __init__(self, dims, schedule, tensors):
        self.d = dims_from(dims)
        self.schedule = np.asarray(schedule, np.uint8)
        self.keep = []
        t = tensors

        def get(name):
            arr = np.ascontiguousarray(t[name][2])
            self.keep.append(arr)
            return c_void_p(arr.ctypes.data)

        n = self.d.n_layers
        self.layers = (Layer * n)()
        for i in range(n):
            p = f"model.language_model.layers.{i}."
            L = self.layers[i]
            L.is_linear = int(self.schedule[i])
            L.gate_up, L.down = get(p + "mlp.gate_up_proj.weight"), get(p + "mlp.down_proj.weight")
            L.input_norm, L.post_norm = get(p + "input_layernorm.weight"), get(p + "post_attention_layernorm.weight")
            if L.is_linear:
                L.in_proj, L.out_proj = get(p + "linear_attn.in_proj_all.weight"), get(p + "linear_attn.out_proj.weight")
                L.conv_w, L.lin_norm = get(p + "linear_attn.conv1d.weight"), get(p + "linear_attn.norm.weight")
                L.a_log, L.dt_bias = get(p + "linear_attn.A_log"), get(p + "linear_attn.dt_bias")
                ba = p + "linear_attn.in_proj_ba.weight"
                if ba in t:  # Q8 gate rows (weights.inl:1700-1747)
                    blocks8 = np.ascontiguousarray(t[ba][2]).view(Q8_0).reshape(-1)
                    sc = blocks8["d"].view(np.float16).astype(np.float32)
                    self.keep.append(sc)
                    L.gate_rows, L.gate_q8, L.gate_scales = int(t[ba][1][0]), get(ba), c_void_p(sc.ctypes.data)
            else:
                L.in_proj, L.out_proj = get(p + "self_attn.qkv_proj.weight"), get(p + "self_attn.o_proj.weight")
                L.q_norm, L.k_norm = get(p + "self_attn.q_norm.weight"), get(p + "self_attn.k_norm.weight")
        emb = "model.language_model.embed_tokens.weight"
        g16 = t[emb][0] == 8  # q4_g16_cpu_dot4
        self.w = Weights(None if g16 else get(emb), get(emb) if g16 else None,
                         get("model.language_model.norm.weight"), self.layers)

    def linear_row(self, layer, conv_state, ring, recurrent, projected):
        """run_linear_attention_step for one row from given inputs: returns
        (core, conv_state, ring, recurrent) after the step (inputs are copied)."""
        d = self.d
        conv = np.array(conv_state, np.float32).ravel()
        rec = np.array(recurrent, np.float32).ravel()
        proj = np.ascontiguousarray(projected, np.float32)
        core = np.zeros(d.lin_v_heads * d.lin_v_dim, np.float32)
        r = c_size_t(int(ring))
        rc = lib.q35o_linear_attention_row(ctypes.byref(self.d), ctypes.byref(self.layers[layer]), ptr(conv),
                                           ctypes.byref(r), ptr(rec), ptr(proj), ptr(core))
        assert rc == 0
        return core, conv, r.value, rec

    def full_row(self, layer, keys, values, position, projected):
        """prepare_full_attention_row + run_full_attention_step for one row:
        keys/values [position + 1][kv_width] binary16 (the row at `position`
        is written); returns (core, keys, values)."""
        d = self.d
        half = d.rope_dim // 2
        cs = np.zeros((position + 1) * half, np.float32)
        sn = np.zeros_like(cs)
        lib.q35o_rope_tables(c_float(d.rope_theta), d.rope_dim, position + 1, ptr(cs), ptr(sn))
        k = np.array(keys, np.uint16).ravel()
        v = np.array(values, np.uint16).ravel()
        proj = np.ascontiguousarray(projected, np.float32)
        core = np.zeros(d.n_heads * d.head_dim, np.float32)
        rc = lib.q35o_full_attention_row(ctypes.byref(self.d), ctypes.byref(self.layers[layer]), ptr(k), ptr(v),
                                         position, ptr(cs[position * half:]), ptr(sn[position * half:]), ptr(proj),
                                         ptr(core))
        assert rc == 0
        return core, k, v

    def new_state(self, capacity, prompt):
        d = self.d
        nlin = int(self.schedule.sum())
        nfull = d.n_layers - nlin
        ch = 2 * d.lin_k_heads * d.lin_k_dim + d.lin_v_heads * d.lin_v_dim
        st = {
            "conv": [np.zeros((d.lin_kernel - 1) * ch, np.float32) for _ in range(nlin)],
            "rec": [np.zeros(d.lin_v_heads * d.lin_v_dim * d.lin_k_dim, np.float32) for _ in range(nlin)],
            "keys": [np.zeros(capacity * d.n_kv_heads * d.head_dim, np.uint16) for _ in range(nfull)],
            "values": [np.zeros(capacity * d.n_kv_heads * d.head_dim, np.uint16) for _ in range(nfull)],
            "ring": np.zeros(max(nlin, 1), np.uint64),
            "counts": np.zeros(d.vocab, np.int32),
        }
        for tok in prompt:
            st["counts"][tok] += 1

        def arr(lst):
            return (P * max(len(lst), 1))(*[c_void_p(a.ctypes.data) for a in lst])

        s = State(arr(st["conv"]), st["ring"].ctypes.data_as(POINTER(c_size_t)), arr(st["rec"]),
                  arr(st["keys"]), arr(st["values"]), st["counts"].ctypes.data_as(POINTER(c_int)), 0, capacity)
        st["struct"] = s
        return st

    def step(self, states, tokens, penalty=1.0, want_logits=False):
        b = len(states)
        arr = (POINTER(State) * b)(*[ctypes.pointer(s["struct"]) for s in states])
        toks = np.ascontiguousarray(tokens, np.int32)
        out = np.zeros(b, np.int32)
        logits = np.zeros((b, self.d.vocab), np.float32) if want_logits else None
        hidden = np.zeros((b, self.d.hidden), np.float32)
        rc = lib.q35o_forward_batch(ctypes.byref(self.d), ctypes.byref(self.w), arr, ptr(toks), b, penalty,
                                    ptr(out), ptr(logits), ptr(hidden))
        assert rc == 0
        return out, logits, hidden


# ------------------------------------------------------------ reference build

def ref_available():
    return os.path.exists(REF_SO)


_ref = None


def ref():
    """ctypes handle of oracle/_ref/libq35ref.so (the reference C++ build)."""
    global _ref
    if _ref is None:
        r = ctypes.CDLL(REF_SO)
        sigs = {
            "ref_backend_resolve": (c_int, [c_int]),
            "ref_backend_name": (ctypes.c_char_p, [c_int]),
            "ref_float_to_half": (c_uint16, [c_float]),
            "ref_half_to_float": (c_float, [c_uint16]),
            "ref_q8_0_quantize_vector_1": (None, [P, P, c_size_t, c_int]),
            "ref_q8_0_quantize_vectors_4": (None, [P, P, c_size_t, c_size_t, c_int]),
            "ref_q4_h128_prepare_activation_1": (c_int, [P, P, c_size_t, c_uint64, c_int]),
            "ref_q4_h128_prepare_activations_4": (c_int, [P, P, c_size_t, c_size_t, c_uint64, c_int]),
            "ref_q4_h128_transform_block": (None, [P, P, c_size_t, c_uint64]),
            "ref_q4_h128_quantize_matrix": (c_int, [P, P, c_size_t, c_size_t, c_uint64]),
            "ref_q4_h128_quantize_transformed": (None, [P, P, c_size_t]),
            "ref_q4_dot4_pack_rows_8": (None, [P, P, c_size_t, c_size_t]),
            "ref_q4_dot4_unpack_rows_8": (None, [P, P, c_size_t, c_size_t]),
            "ref_q4_dot4_dequantize_row": (None, [P, c_size_t, P, c_size_t]),
            "ref_q4_dot4_matvec": (None, [P, P, P, c_size_t, c_size_t, c_int]),
            "ref_q4_dot4_matmul": (None, [P, P, P, c_size_t, c_size_t, c_size_t, c_size_t, c_int]),
            "ref_q4_dot4_argmax": (None, [P, P, P, c_float, c_size_t, c_size_t, c_size_t, c_int, P, P]),
            "ref_gated_delta_net_update_rows": (None, [P, P, P, P, P, P, P, c_size_t, c_size_t, c_size_t, c_size_t,
                                                       c_size_t, c_int]),
            "ref_causal_attention_decode_gqa_pairs": (None, [P, P, P, P, P, P, c_size_t, c_size_t, c_size_t, c_int,
                                                             c_int, c_int, c_int, c_float, c_size_t, c_size_t, c_int]),
            "ref_attention_cache_store_f16": (None, [P, P, c_size_t, c_int]),
            "ref_add_f32": (None, [P, P, P, c_size_t, c_int]),
            "ref_rope_f32": (None, [P, c_size_t, c_size_t, c_size_t, P, P, c_int]),
            "ref_causal_conv1d_silu_f32": (None, [P, c_size_t, P, c_size_t, P, P, c_size_t, c_size_t, c_size_t, c_int]),
            "ref_rms_norm_f32": (None, [P, P, P, c_size_t, c_size_t, c_float, c_float, c_int]),
            "ref_l2_normalize_f32": (None, [P, c_size_t, c_size_t, c_float, c_float, c_int]),
            "ref_silu_mul_f32": (None, [P, P, P, c_size_t, c_int]),
            "ref_q4_g16_dequantize_row": (None, [P, c_size_t, P, c_size_t]),
            "ref_q4_g16_matvec": (None, [P, P, P, c_size_t, c_size_t, c_int]),
            "ref_q4_g16_pack_activations": (None, [P, P, c_size_t, c_size_t]),
            "ref_q4_g16_matmul": (None, [P, P, P, c_size_t, c_size_t, c_size_t, c_size_t, c_int]),
            "ref_q8_0_matmul": (None, [P, P, P, c_size_t, c_size_t, c_size_t, c_size_t, c_int, P]),
            "ref_engine_set_probe": (None, [P, c_size_t, P]),
            "ref_engine_sample": (c_int, [ctypes.c_char_p, ctypes.c_char_p, c_int, P, c_size_t, c_size_t, c_float,
                                          c_float, c_int, c_float, ctypes.c_int64, P, P, c_size_t, ctypes.c_char_p,
                                          c_size_t]),
            "ref_engine_greedy": (c_int, [ctypes.c_char_p, ctypes.c_char_p, c_int, c_int, P, c_size_t, c_size_t, c_size_t,
                                          c_float, P, P, P, P, P, ctypes.c_char_p, c_size_t]),
            "ref_executor_create": (P, [c_size_t]),
            "ref_executor_destroy": (None, [P]),
            "ref_executor_threads": (c_size_t, [P]),
            "ref_par_q4_dot4": (c_int, [P, P, P, P, c_size_t, c_size_t, c_size_t, c_int]),
            "ref_par_delta": (c_int, [P, P, P, P, P, P, P, P, c_size_t, c_size_t, c_size_t, c_size_t, c_int]),
            "ref_par_attention": (c_int, [P, P, P, P, P, P, P, P, c_size_t, c_size_t, c_int, c_int, c_int, c_float,
                                          c_int]),
            "ref_engine_mixed": (c_int, [ctypes.c_char_p, ctypes.c_char_p, c_int, P, c_size_t, c_size_t, P, c_size_t,
                                         c_size_t, P, P, P, ctypes.c_char_p, c_size_t]),
        }
        for name, (res, args) in sigs.items():
            f = getattr(r, name)
            f.restype, f.argtypes = res, args
        _ref = r
    return _ref


def ref_engine_sample(model_dir, artifact, prompt, new_tokens, vocab, temperature, top_p, top_k, penalty, seed,
                      threads=8):
    """One sampled request through the reference CpuEngine (oracle/_ref):
    returns (tokens [new_tokens], raw logits [new_tokens][vocab]) as its
    logits callback saw them."""
    prompt = np.ascontiguousarray(prompt, np.int32)
    out = np.zeros(new_tokens, np.int32)
    logits = np.zeros((new_tokens, vocab), np.float32)
    err = ctypes.create_string_buffer(512)
    rc = ref().ref_engine_sample(os.fsencode(model_dir), os.fsencode(artifact), threads, prompt.ctypes.data,
                                 prompt.size, new_tokens, temperature, top_p, top_k, penalty, seed, out.ctypes.data,
                                 logits.ctypes.data, vocab, err, 512)
    if rc != 0:
        raise RuntimeError(err.value.decode())
    return out, logits
