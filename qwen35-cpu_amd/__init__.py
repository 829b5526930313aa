"""Python binding of the MI355X (gfx950) decode backend, libq35hip.so.

Mirrors the reference's operator surface -- the free functions of
include/qwen35x/cpu/*.h and the CpuEngine API of
include/qwen35x/runtime/cpu_engine.h -- over the C ABI declared in
include/q35_hip.h. There is no CPU fallback: importing this module without a
built libq35hip.so raises, and every call runs the HIP kernels.

The directory name is not a Python identifier; load it as
``importlib`` module ``qwen35_cpu_amd`` (see ``load()`` in __graft_entry__.py).
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_size_t, c_uint8, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libq35hip.so")

Q35_OK = 0
STATUS = {0: "ok", 1: "invalid argument", 2: "HIP runtime error", 3: "out of memory",
          4: "invalid state", 5: "unsupported shape", 6: "I/O error"}
REQ_STATUS = {0: "prefill", 1: "decode", 2: "complete", 3: "cancelled", 4: "failed", 5: "queued"}
REQ_STATUS_INV = {v: k for k, v in REQ_STATUS.items()}
ENC_F32, ENC_Q4_0_DOT4, ENC_Q4_H128_DOT4 = 0, 5, 6
# kernel classes of the step profiler (q35_runtime_profile_read)
KERNEL_CLASSES = ("embed", "prep", "gemm", "delta", "attn_prep", "attention", "argmax", "head")
DEFAULT_SIGN_SEED = 0x5148333548313238  # q4_h128.h:25-26

Q4X8_BYTES, Q8X4_BYTES, Q8X1_BYTES = 144, 152, 40

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
        "(there is no CPU fallback for the MI355X backend)")
lib = ctypes.CDLL(LIB_PATH)


class Q35Error(RuntimeError):
    pass


class ModelDims(ctypes.Structure):
    """RuntimeDims (src/runtime/weights.inl:336-357)."""
    _fields_ = [("n_layers", c_int32), ("hidden", c_int32), ("intermediate", c_int32), ("vocab", c_int32),
                ("n_heads", c_int32), ("n_kv_heads", c_int32), ("head_dim", c_int32), ("rope_dim", c_int32),
                ("rope_theta", c_float), ("rms_eps", c_float),
                ("lin_kernel", c_int32), ("lin_k_heads", c_int32), ("lin_v_heads", c_int32),
                ("lin_k_dim", c_int32), ("lin_v_dim", c_int32), ("sign_seed", c_uint64)]

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_}


class RuntimeConfig(ctypes.Structure):
    _fields_ = [("max_slots", c_int32), ("max_batch", c_int32), ("max_context", c_int32),
                ("page_tokens", c_int32), ("total_pages", c_int32), ("use_graphs", c_int32),
                ("max_step_rows", c_int32)]


class Segment(ctypes.Structure):
    """q35_segment: consecutive positions of one request in a packed step."""
    _fields_ = [("slot", c_int32), ("pos0", c_int32), ("count", c_int32), ("tokens", POINTER(c_int32)),
                ("page_table", POINTER(c_int32)), ("max_pages", c_int32), ("penalty", c_float),
                ("count_input", c_uint8), ("want_token", c_uint8)]


class StepDesc(ctypes.Structure):
    _fields_ = [("batch", c_int32), ("slots", POINTER(c_int32)), ("positions", POINTER(c_int32)),
                ("tokens", POINTER(c_int32)), ("count_input", POINTER(c_uint8)),
                ("penalties", POINTER(c_float)), ("page_table", POINTER(c_int32)), ("max_pages", c_int32)]


class EngineConfig(ctypes.Structure):
    _fields_ = [("max_resident_requests", c_int32), ("max_context", c_int32),
                ("max_decode_batch_size", c_int32), ("prefill_chunk_size", c_int32),
                ("page_tokens", c_int32), ("use_graphs", c_int32), ("max_prefix_bytes", c_uint64),
                ("max_prefill_requests", c_int32), ("packed_steps", c_int32),
                ("max_queued_requests", c_int32), ("max_buffered_tokens", c_int32)]


class EngineStats(ctypes.Structure):
    """q35_engine_stats (CpuEngineStats, cpu_engine.h:151-168)."""
    _fields_ = [(n, c_uint64) for n in (
        "batch_ticks", "batch_rows", "projection_batches", "lm_head_batches", "greedy_lm_head_batches",
        "state_batches", "shared_prefill_ticks", "shared_prefill_requests", "packed_ticks", "packed_rows",
        "queued_requests", "resident_requests", "physical_kv_bytes")]


class RequestResult(ctypes.Structure):
    _fields_ = [("status", c_int32), ("generated_tokens", c_uint64), ("committed_tokens", c_uint64),
                ("prefill_tokens", c_uint64), ("decode_forwards", c_uint64),
                ("prefill_ms", c_double), ("decode_ms", c_double),
                ("cached_prefix_tokens", c_uint64), ("prefix_restore_ms", c_double),
                ("queue_ms", c_double), ("prefix_written_tokens", c_uint64)]


class Candidate(ctypes.Structure):
    _fields_ = [("value", c_float), ("token", c_int32)]


class RowSampling(ctypes.Structure):
    _fields_ = [("top_k", c_int32), ("inv_temperature", c_float)]


MAX_CANDIDATES = 64
# q35_logits_callback: (context, index, forced_token, logits, count) -> nonzero to continue
LOGITS_CALLBACK = ctypes.CFUNCTYPE(c_int, c_void_p, c_size_t, c_int32, POINTER(c_float), c_size_t)


class RequestSpec(ctypes.Structure):
    _fields_ = [("prompt_tokens", POINTER(c_int32)), ("prompt_count", c_size_t), ("max_new_tokens", c_size_t),
                ("temperature", c_float), ("top_p", c_float), ("top_k", c_int32),
                ("repetition_penalty", c_float), ("seed", ctypes.c_int64),
                ("stop_token_ids", POINTER(c_int32)), ("stop_count", c_size_t),
                ("stop_sequences", POINTER(c_int32)), ("stop_sequence_lengths", POINTER(c_size_t)),
                ("stop_sequence_count", c_size_t),
                ("forced_output_tokens", POINTER(c_int32)), ("forced_count", c_size_t),
                ("logits_callback", LOGITS_CALLBACK), ("logits_callback_context", c_void_p),
                ("prefix", c_uint64), ("sampling_constraint", c_void_p),
                ("selected_logit_tokens", POINTER(c_int32)), ("selected_logit_count", c_size_t),
                ("selected_logits_callback", LOGITS_CALLBACK), ("selected_logits_callback_context", c_void_p),
                ("register_prefix_tokens", c_uint64), ("trust_namespace", c_char_p)]


CONSTRAINT_APPLY = ctypes.CFUNCTYPE(c_int, c_void_p, POINTER(c_float), c_size_t)
CONSTRAINT_ACCEPT = ctypes.CFUNCTYPE(c_int, c_void_p, c_int32)


class SamplingConstraint(ctypes.Structure):
    """q35_sampling_constraint (CpuSamplingConstraint, cpu_engine.h:84-94)."""
    _fields_ = [("context", c_void_p), ("apply", CONSTRAINT_APPLY), ("accept", CONSTRAINT_ACCEPT)]


class PrefixStats(ctypes.Structure):
    _fields_ = [("prefix_builds", c_uint64), ("prefix_build_fallbacks", c_uint64), ("prefix_hits", c_uint64),
                ("prefix_cached_tokens", c_uint64), ("prefix_evictions", c_uint64), ("prefix_entries", c_uint64),
                ("prefix_bytes", c_uint64)]


# Stage trace points (include/q35_hip.h, Q35_TRACE_*), in enum order.
TRACE_POINTS = ["X_IN", "NORMED_IN", "CODES_IN", "SCALES_IN", "GATES", "PROJ_IN", "STATE_BEFORE", "STATE_AFTER",
                "CONV_BEFORE", "CONV_AFTER", "CORE", "CODES_CORE", "SCALES_CORE", "Q_ROT", "ATTN_GATE", "K_POOL",
                "V_POOL", "PROJ_OUT", "X_MID", "NORMED_POST", "CODES_POST", "SCALES_POST", "GATE_UP", "SILU",
                "CODES_DOWN", "SCALES_DOWN", "DOWN", "X_FINAL", "HIDDEN", "CODES_HEAD", "SCALES_HEAD"]
TRACE = {name: i for i, name in enumerate(TRACE_POINTS)}

P = c_void_p
_SIGS = {
    "q35_context_create": (c_int, [c_int, P, POINTER(P)]),
    "q35_context_destroy": (None, [P]),
    "q35_context_synchronize": (c_int, [P]),
    "q35_context_stream": (P, [P]),
    "q35_context_last_error": (c_char_p, [P]),
    "q35_status_string": (c_char_p, [c_int]),
    "q35_context_device_info": (c_int, [P, POINTER(c_int), c_char_p, c_size_t]),
    "q35_device_alloc": (c_int, [P, c_size_t, POINTER(P)]),
    "q35_device_free": (c_int, [P, P]),
    "q35_memcpy_h2d": (c_int, [P, P, P, c_size_t]),
    "q35_memcpy_d2h": (c_int, [P, P, P, c_size_t]),
    "q35_memcpy_d2d": (c_int, [P, P, P, c_size_t]),
    "q35_memset_device": (c_int, [P, P, c_int, c_size_t]),
    "q35_timer_begin": (c_int, [P]),
    "q35_timer_end": (c_int, [P, POINTER(c_double)]),
    "q35_q8_0_quantize_vector_1": (c_int, [P, P, P, c_size_t]),
    "q35_q8_0_quantize_vectors_4": (c_int, [P, P, P, c_size_t, c_size_t]),
    "q35_q4_h128_prepare_activation_1": (c_int, [P, P, P, c_size_t, c_uint64]),
    "q35_q4_h128_prepare_activations_4": (c_int, [P, P, P, c_size_t, c_size_t, c_uint64]),
    "q35_q4_dot4_matvec": (c_int, [P, P, P, P, c_size_t, c_size_t]),
    "q35_q4_dot4_matmul": (c_int, [P, P, P, P, c_size_t, c_size_t, c_size_t, c_size_t]),
    "q35_q4_dot4_matmul_exact": (c_int, [P, P, P, P, c_size_t, c_size_t, c_size_t, c_size_t]),
    "q35_q4_dot4_matmul_noalloc": (c_int, [P, P, P, P, c_size_t, c_size_t, c_size_t, c_size_t]),
    "q35_q4_dot4_matmul_x1": (c_int, [P, P, P, P, c_size_t, c_size_t, c_size_t, c_size_t]),
    "q35_q4_dot4_has_x1_tile": (c_int, [c_size_t]),
    "q35_q4_dot4_block_dots": (c_int, [P, P, P, P, c_size_t, c_size_t, c_size_t]),
    "q35_q4_dot4_argmax_batch": (c_int, [P, P, P, P, P, c_size_t, c_size_t, c_size_t, P, P]),
    "q35_gated_delta_net_update_rows": (c_int, [P, P, P, P, P, P, P, P, c_size_t, c_size_t, c_size_t,
                                                c_size_t, c_size_t]),
    "q35_gated_delta_net_update_batch": (c_int, [P, P, P, P, P, P, P, P, c_size_t, c_size_t, c_size_t,
                                                 c_size_t]),
    "q35_attention_decode_paged": (c_int, [P, P, P, P, P, P, c_size_t, P, c_size_t, P, c_size_t, c_int,
                                           c_int, c_int, c_float]),
    "q35_attention_cache_store_f16": (c_int, [P, P, P, c_size_t]),
    "q35_rms_norm_f32": (c_int, [P, P, P, P, c_size_t, c_size_t, c_float, c_float]),
    "q35_l2_normalize_f32": (c_int, [P, P, c_size_t, c_size_t, c_float, c_float]),
    "q35_causal_conv1d_silu_f32": (c_int, [P, P, c_size_t, P, c_size_t, P, P, c_size_t, c_size_t, c_size_t,
                                           c_size_t, c_size_t]),
    "q35_silu_mul_f32": (c_int, [P, P, P, P, c_size_t]),
    "q35_rope_f32": (c_int, [P, P, c_size_t, c_size_t, c_size_t, P, P]),
    "q35_model_create": (c_int, [P, POINTER(ModelDims), P, POINTER(P)]),
    "q35_model_upload_tensor": (c_int, [P, c_char_p, c_int, POINTER(c_uint64), c_size_t, P, c_size_t]),
    "q35_model_finalize": (c_int, [P]),
    "q35_model_destroy": (None, [P]),
    "q35_model_load_artifact": (c_int, [P, c_char_p, POINTER(ModelDims), P, POINTER(P)]),
    "q35_model_dims_preset": (c_int, [c_int, POINTER(ModelDims), P, c_size_t]),
    "q35_write_random_artifact": (c_int, [c_char_p, POINTER(ModelDims), P, c_uint64, c_float]),
    "q35_write_random_artifact_ex": (c_int, [c_char_p, POINTER(ModelDims), P, c_uint64, c_float, ctypes.c_uint32]),
    "q35_random_weight_rows": (c_int, [c_char_p, c_uint64, c_uint64, c_uint64, c_uint64, c_float, P]),
    "q35_runtime_create": (c_int, [P, POINTER(RuntimeConfig), POINTER(P)]),
    "q35_runtime_destroy": (None, [P]),
    "q35_slot_alloc": (c_int, [P, P, c_size_t, POINTER(c_int32)]),
    "q35_slot_free": (c_int, [P, c_int32]),
    "q35_page_alloc": (c_int, [P, POINTER(c_int32)]),
    "q35_page_retain": (c_int, [P, c_int32]),
    "q35_page_release": (c_int, [P, c_int32]),
    "q35_page_copy": (c_int, [P, c_int32, c_int32, c_int32]),
    "q35_page_refcount": (c_int, [P, c_int32]),
    "q35_runtime_free_pages": (c_int, [P]),
    "q35_runtime_step": (c_int, [P, POINTER(StepDesc), P, P]),
    "q35_runtime_prefill": (c_int, [P, c_int32, c_int32, P, c_int32, P, c_int32, c_float, P]),
    "q35_runtime_step_segments": (c_int, [P, P, c_int32, P, P, P, P]),
    "q35_runtime_last_hidden": (c_int, [P, P, c_size_t]),
    "q35_runtime_set_profiling": (c_int, [P, c_int]),
    "q35_runtime_set_trace": (c_int, [P, c_int]),
    "q35_runtime_set_fused": (c_int, [P, c_int]),
    "q35_runtime_trace_read": (c_int, [P, c_int, c_int, P, c_size_t, POINTER(c_size_t)]),
    "q35_runtime_profile_reset": (c_int, [P]),
    "q35_runtime_profile_read": (c_int, [P, c_int, POINTER(c_double), POINTER(c_uint64), POINTER(c_double)]),
    "q35_runtime_set_step_timing": (c_int, [P, c_int]),
    "q35_runtime_step_timing_read": (c_int, [P, POINTER(c_double), POINTER(c_uint64)]),
    "q35_engine_create": (c_int, [P, POINTER(EngineConfig), POINTER(P)]),
    "q35_engine_destroy": (None, [P]),
    "q35_engine_submit": (c_int, [P, P, c_size_t, c_size_t, c_float, P, c_size_t, POINTER(c_uint64)]),
    "q35_engine_advance": (c_int, [P, c_uint64]),
    "q35_engine_advance_batch": (c_int, [P, P, c_size_t]),
    "q35_engine_step": (c_int, [P, POINTER(c_int32)]),
    "q35_engine_read_output": (c_int, [P, c_uint64, c_size_t, P, POINTER(c_size_t)]),
    "q35_prefill_chunk_token_count": (c_size_t, [c_size_t, c_size_t, c_size_t]),
    "q35_engine_prefill_batch": (c_int, [P, P, c_size_t]),
    "q35_engine_result": (c_int, [P, c_uint64, POINTER(RequestResult), P, c_size_t, POINTER(c_size_t)]),
    "q35_engine_cancel": (c_int, [P, c_uint64]),
    "q35_engine_release": (c_int, [P, c_uint64]),
    "q35_engine_last_error": (c_char_p, [P]),
    "q35_engine_runtime": (P, [P]),
    "q35_engine_register_prefix": (c_int, [P, P, c_size_t, c_char_p, POINTER(c_uint64)]),
    "q35_engine_find_prefix": (c_int, [P, P, c_size_t, c_char_p, POINTER(c_uint64), POINTER(c_size_t)]),
    "q35_engine_release_prefix": (c_int, [P, c_uint64]),
    "q35_engine_submit_prefixed": (c_int, [P, P, c_size_t, c_size_t, c_float, P, c_size_t, c_uint64,
                                           POINTER(c_uint64)]),
    "q35_engine_prefix_stats": (c_int, [P, POINTER(PrefixStats)]),
    "q35_engine_get_stats": (c_int, [P, POINTER(EngineStats)]),
    "q35_runtime_head": (c_int, [P, c_int32, P, c_float, P]),
    "q35_runtime_step_candidates": (c_int, [P, POINTER(StepDesc), P, P, P]),
    "q35_runtime_head_candidates": (c_int, [P, c_int32, P, c_float, P, P, P]),
    "q35_slot_counts": (c_int, [P, c_int32, P, c_size_t]),
    "q35_engine_submit_spec": (c_int, [P, POINTER(RequestSpec), POINTER(c_uint64)]),
    "q35_state_snapshot_create": (c_int, [P, c_int32, c_int32, P, POINTER(P)]),
    "q35_state_snapshot_restore": (c_int, [P, P, c_int32]),
    "q35_state_snapshot_tokens": (c_int32, [P]),
    "q35_state_snapshot_bytes": (c_size_t, [P]),
    "q35_state_snapshot_hidden": (c_int, [P, P, c_size_t]),
    "q35_state_snapshot_destroy": (None, [P]),
}
for _name, (_res, _args) in _SIGS.items():
    _f = getattr(lib, _name)
    _f.restype = _res
    _f.argtypes = _args


def _ptr(a):
    """Host numpy array -> void*."""
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def model_dims(preset: int = 0):
    """Dims + attention schedule of the reference shapes: 0 = 0.8B, 1 = 2B, 2 = 4B."""
    d = ModelDims()
    sched = np.zeros(64, np.uint8)
    _check(lib.q35_model_dims_preset(preset, ctypes.byref(d), _ptr(sched), 64), "dims preset")
    return d, sched[: d.n_layers].copy()


def _check(status, what, ctx=None):
    if status != Q35_OK:
        detail = ""
        if ctx is not None:
            detail = lib.q35_context_last_error(ctx).decode(errors="replace")
        raise Q35Error(f"{what}: {STATUS.get(status, status)} {detail}".strip())


class DeviceArray:
    """A device allocation with its host-side shape/dtype."""

    def __init__(self, ctx: "Context", shape, dtype):
        self.ctx, self.shape, self.dtype = ctx, tuple(shape), np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize if self.shape else self.dtype.itemsize
        p = c_void_p()
        _check(lib.q35_device_alloc(ctx.handle, max(self.nbytes, 1), ctypes.byref(p)), "device alloc", ctx.handle)
        self.ptr = p

    @property
    def address(self):
        return self.ptr.value

    def upload(self, host):
        host = np.ascontiguousarray(host, dtype=self.dtype)
        assert host.nbytes == self.nbytes, (host.nbytes, self.nbytes)
        _check(lib.q35_memcpy_h2d(self.ctx.handle, self.ptr, _ptr(host), host.nbytes), "h2d", self.ctx.handle)
        return self

    def download(self):
        out = np.empty(self.shape, self.dtype)
        _check(lib.q35_memcpy_d2h(self.ctx.handle, _ptr(out), self.ptr, self.nbytes), "d2h", self.ctx.handle)
        return out

    def free(self):
        if self.ptr is not None and self.ptr.value:
            lib.q35_device_free(self.ctx.handle, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    """One device, one stream (replaces the reference CpuExecutor)."""

    def __init__(self, device: int = 0):
        h = c_void_p()
        _check(lib.q35_context_create(device, None, ctypes.byref(h)), "context create")
        self.handle = h

    def device_info(self):
        cu = c_int()
        arch = ctypes.create_string_buffer(64)
        _check(lib.q35_context_device_info(self.handle, ctypes.byref(cu), arch, 64), "device info")
        return cu.value, arch.value.decode()

    def array(self, host=None, shape=None, dtype=None):
        if host is not None:
            host = np.ascontiguousarray(host)
            return DeviceArray(self, host.shape, host.dtype).upload(host)
        return DeviceArray(self, shape, dtype)

    def synchronize(self):
        _check(lib.q35_context_synchronize(self.handle), "synchronize", self.handle)

    def check(self, status, what):
        _check(status, what, self.handle)

    def timer_begin(self):
        self.check(lib.q35_timer_begin(self.handle), "timer")

    def timer_end(self):
        ms = c_double()
        self.check(lib.q35_timer_end(self.handle, ctypes.byref(ms)), "timer")
        return ms.value

    def close(self):
        if self.handle is not None:
            lib.q35_context_destroy(self.handle)
            self.handle = None


# ------------------------------------------------------------------ operators
# Same names and argument meaning as the reference free functions; buffers are
# DeviceArray objects (device memory), shapes follow the reference layouts.

def q8_0_quantize_vector_1(ctx, x, out, blocks):
    ctx.check(lib.q35_q8_0_quantize_vector_1(ctx.handle, x.ptr, out.ptr, blocks), "q8_0_quantize_vector_1")


def q8_0_quantize_vectors_4(ctx, x, out, vectors, blocks):
    ctx.check(lib.q35_q8_0_quantize_vectors_4(ctx.handle, x.ptr, out.ptr, vectors, blocks), "q8_0_quantize_vectors_4")


def q4_h128_prepare_activation_1(ctx, x, out, columns, seed=DEFAULT_SIGN_SEED):
    ctx.check(lib.q35_q4_h128_prepare_activation_1(ctx.handle, x.ptr, out.ptr, columns, seed),
              "q4_h128_prepare_activation_1")


def q4_h128_prepare_activations_4(ctx, x, out, vectors, columns, seed=DEFAULT_SIGN_SEED):
    ctx.check(lib.q35_q4_h128_prepare_activations_4(ctx.handle, x.ptr, out.ptr, vectors, columns, seed),
              "q4_h128_prepare_activations_4")


def q4_dot4_matvec(ctx, m, v, out, rows, blocks):
    ctx.check(lib.q35_q4_dot4_matvec(ctx.handle, m.ptr, v.ptr, out.ptr, rows, blocks), "q4_dot4_matvec")


def q4_dot4_matmul(ctx, m, v, out, rows, count, blocks, stride, exact=False):
    f = lib.q35_q4_dot4_matmul_exact if exact else lib.q35_q4_dot4_matmul
    ctx.check(f(ctx.handle, m.ptr, v.ptr, out.ptr, rows, count, blocks, stride), "q4_dot4_matmul")


def q4_dot4_matmul_noalloc(ctx, m, v, out, rows, count, blocks, stride):
    """q4_dot4_matmul through the entry point that allocates nothing (its
    scratch is a fixed 16 MiB device array shared by every call on the GPU)."""
    ctx.check(lib.q35_q4_dot4_matmul_noalloc(ctx.handle, m.ptr, v.ptr, out.ptr, rows, count, blocks, stride),
              "q4_dot4_matmul_noalloc")


def q4_dot4_matmul_x1(ctx, m, v, out, rows, count, blocks, stride):
    """q4_dot4_matmul_x1: independently prepared X1 rows [count][blocks]."""
    ctx.check(lib.q35_q4_dot4_matmul_x1(ctx.handle, m.ptr, v.ptr, out.ptr, rows, count, blocks, stride),
              "q4_dot4_matmul_x1")


def q4_dot4_block_dots(ctx, m, v, out, rows, count, blocks):
    ctx.check(lib.q35_q4_dot4_block_dots(ctx.handle, m.ptr, v.ptr, out.ptr, rows, count, blocks),
              "q4_dot4_block_dots")


def q4_dot4_argmax_batch(ctx, m, v, counts, penalties, rows, count, blocks, out_index, out_value):
    ctx.check(lib.q35_q4_dot4_argmax_batch(ctx.handle, m.ptr, v.ptr, counts.ptr if counts else None,
                                           penalties.ptr if penalties else None, rows, count, blocks,
                                           out_index.ptr, out_value.ptr if out_value else None),
              "q4_dot4_argmax_batch")


def gated_delta_net_update_rows(ctx, state, q, k, v, alpha, beta, out, heads, kdim, vdim, begin, end):
    ctx.check(lib.q35_gated_delta_net_update_rows(ctx.handle, state.ptr, q.ptr, k.ptr, v.ptr, alpha.ptr, beta.ptr,
                                                  out.ptr, heads, kdim, vdim, begin, end),
              "gated_delta_net_update_rows")


def gated_delta_net_update_batch(ctx, state_ptrs, q, k, v, alpha, beta, out, batch, heads, kdim, vdim):
    ctx.check(lib.q35_gated_delta_net_update_batch(ctx.handle, state_ptrs.ptr, q.ptr, k.ptr, v.ptr, alpha.ptr,
                                                   beta.ptr, out.ptr, batch, heads, kdim, vdim),
              "gated_delta_net_update_batch")


def attention_decode_paged(ctx, q, gates, k_pool, v_pool, page_table, max_pages, seq_lens, page_tokens, out,
                           batch, heads, kv_heads, head_dim, scale):
    ctx.check(lib.q35_attention_decode_paged(ctx.handle, q.ptr, gates.ptr, k_pool.ptr, v_pool.ptr, page_table.ptr,
                                             max_pages, seq_lens.ptr, page_tokens, out.ptr, batch, heads, kv_heads,
                                             head_dim, scale), "attention_decode_paged")


def attention_cache_store_f16(ctx, x, out, count):
    ctx.check(lib.q35_attention_cache_store_f16(ctx.handle, x.ptr, out.ptr, count), "attention_cache_store_f16")


def rms_norm_f32(ctx, x, w, out, rows, width, eps, offset):
    ctx.check(lib.q35_rms_norm_f32(ctx.handle, x.ptr, w.ptr, out.ptr, rows, width, eps, offset), "rms_norm_f32")


def l2_normalize_f32(ctx, x, rows, width, eps, scale=1.0):
    ctx.check(lib.q35_l2_normalize_f32(ctx.handle, x.ptr, rows, width, eps, scale), "l2_normalize_f32")


def causal_conv1d_silu_f32(ctx, state, ring, x, w, out, channels, kernel, batch=1, input_stride=None,
                           channel_begin=0, channel_end=None):
    ctx.check(lib.q35_causal_conv1d_silu_f32(ctx.handle, state.ptr, ring, x.ptr,
                                             channels if input_stride is None else input_stride, w.ptr, out.ptr,
                                             batch, channels, kernel, channel_begin,
                                             channels if channel_end is None else channel_end),
              "causal_conv1d_silu_f32")


def silu_mul_f32(ctx, g, u, out, count):
    ctx.check(lib.q35_silu_mul_f32(ctx.handle, g.ptr, u.ptr, out.ptr, count), "silu_mul_f32")


def rope_f32(ctx, x, heads, head_dim, rope_dim, cos, sin):
    ctx.check(lib.q35_rope_f32(ctx.handle, x.ptr, heads, head_dim, rope_dim, cos.ptr, sin.ptr), "rope_f32")


# --------------------------------------------------------------- model level

def write_random_artifact(path, dims, schedule, seed=1, weight_std=0.02, head_g16=False, q8_gates=False):
    """Random-init Q35H128 artifact (weights ~N(0, weight_std) through the H128/Q4 packer);
    head_g16 / q8_gates select the optional encodings (G16 tied head, Q8_0 gate rows)."""
    sched = np.ascontiguousarray(schedule, np.uint8)
    flags = (1 if head_g16 else 0) | (2 if q8_gates else 0)
    _check(lib.q35_write_random_artifact_ex(os.fsencode(path), ctypes.byref(dims), _ptr(sched), seed, weight_std,
                                            flags), "write_random_artifact")


def random_weight_rows(name, seed, row0, rows, cols, weight_std=0.02):
    out = np.empty((rows, cols), np.float32)
    _check(lib.q35_random_weight_rows(name.encode(), seed, row0, rows, cols, weight_std, _ptr(out)),
           "random_weight_rows")
    return out


class Model:
    """CpuModel::load equivalent: weights resident in HBM."""

    def __init__(self, ctx, dims, schedule, artifact=None):
        self.ctx, self.dims = ctx, dims
        self.schedule = np.ascontiguousarray(schedule, np.uint8)
        h = c_void_p()
        if artifact is not None:
            ctx.check(lib.q35_model_load_artifact(ctx.handle, os.fsencode(artifact), ctypes.byref(dims),
                                                  _ptr(self.schedule), ctypes.byref(h)), "model load")
        else:
            ctx.check(lib.q35_model_create(ctx.handle, ctypes.byref(dims), _ptr(self.schedule), ctypes.byref(h)),
                      "model create")
        self.handle = h

    def upload(self, name, encoding, shape, payload):
        payload = np.ascontiguousarray(payload)
        shp = (c_uint64 * len(shape))(*shape)
        self.ctx.check(lib.q35_model_upload_tensor(self.handle, name.encode(), encoding, shp, len(shape),
                                                   _ptr(payload), payload.nbytes), "upload " + name)

    def finalize(self):
        self.ctx.check(lib.q35_model_finalize(self.handle), "model finalize")

    def close(self):
        if self.handle is not None:
            lib.q35_model_destroy(self.handle)
            self.handle = None


class _Profiled:
    """Kernel-level timing of the decode step (q35_runtime_set_profiling):
    eager launches, each bracketed by HIP events on the runtime's stream; and
    step timing (q35_runtime_set_step_timing) of the replayed graphs."""

    def _rt(self):
        raise NotImplementedError

    def set_profiling(self, enable=True):
        self.ctx.check(lib.q35_runtime_set_profiling(self._rt(), int(enable)), "set profiling")

    def profile_reset(self):
        self.ctx.check(lib.q35_runtime_profile_reset(self._rt()), "profile reset")

    def set_step_timing(self, enable=True):
        """Step timing (q35_runtime_set_step_timing): each step's launch -- the
        graph replay itself -- between two HIP events; restarts the totals."""
        self.ctx.check(lib.q35_runtime_set_step_timing(self._rt(), int(enable)), "set step timing")

    def step_timing(self):
        """(GPU ms summed over the timed steps, step count)."""
        ms, n = c_double(), c_uint64()
        self.ctx.check(lib.q35_runtime_step_timing_read(self._rt(), ctypes.byref(ms), ctypes.byref(n)),
                       "step timing read")
        return ms.value, n.value

    def profile(self):
        """{class: (total_ms, launches, algorithmic_bytes)}."""
        out = {}
        for i, name in enumerate(KERNEL_CLASSES):
            ms, n, by = c_double(), c_uint64(), c_double()
            self.ctx.check(lib.q35_runtime_profile_read(self._rt(), i, ctypes.byref(ms), ctypes.byref(n),
                                                        ctypes.byref(by)), "profile read")
            out[name] = (ms.value, n.value, by.value)
        return out


class Runtime(_Profiled):
    """Device slots, KV page pool and the captured decode step."""

    def __init__(self, model, max_slots=16, max_batch=16, max_context=1024, page_tokens=16, total_pages=0,
                 use_graphs=True, max_step_rows=0):
        self.model, self.ctx = model, model.ctx
        self.cfg = RuntimeConfig(max_slots, max_batch, max_context, page_tokens, total_pages, int(use_graphs),
                                 int(max_step_rows))
        h = c_void_p()
        self.ctx.check(lib.q35_runtime_create(model.handle, ctypes.byref(self.cfg), ctypes.byref(h)), "runtime create")
        self.handle = h
        self.max_pages = (max_context + page_tokens - 1) // page_tokens

    def slot_alloc(self, prompt):
        prompt = np.ascontiguousarray(prompt, np.int32)
        s = c_int32()
        self.ctx.check(lib.q35_slot_alloc(self.handle, _ptr(prompt), prompt.size, ctypes.byref(s)), "slot alloc")
        return s.value

    def slot_free(self, slot):
        self.ctx.check(lib.q35_slot_free(self.handle, slot), "slot free")

    def page_alloc(self):
        p = c_int32()
        self.ctx.check(lib.q35_page_alloc(self.handle, ctypes.byref(p)), "page alloc")
        return p.value

    def page_release(self, page):
        self.ctx.check(lib.q35_page_release(self.handle, page), "page release")

    def step(self, slots, positions, tokens, page_table, count_input=None, penalties=None, logits=False):
        slots = np.ascontiguousarray(slots, np.int32)
        positions = np.ascontiguousarray(positions, np.int32)
        tokens = np.ascontiguousarray(tokens, np.int32)
        b = slots.size
        table = np.ascontiguousarray(page_table, np.int32).reshape(b, -1)
        ci = np.ascontiguousarray(count_input if count_input is not None else np.zeros(b), np.uint8)
        pen = np.ascontiguousarray(penalties if penalties is not None else np.ones(b), np.float32)
        d = StepDesc(b, slots.ctypes.data_as(POINTER(c_int32)), positions.ctypes.data_as(POINTER(c_int32)),
                     tokens.ctypes.data_as(POINTER(c_int32)), ci.ctypes.data_as(POINTER(c_uint8)),
                     pen.ctypes.data_as(POINTER(c_float)), table.ctypes.data_as(POINTER(c_int32)), table.shape[1])
        out = np.empty(b, np.int32)
        lg = np.empty((b, self.model.dims.vocab), np.float32) if logits else None
        self.ctx.check(lib.q35_runtime_step(self.handle, ctypes.byref(d), _ptr(out), _ptr(lg)), "runtime step")
        return (out, lg) if logits else out

    def step_candidates(self, slots, positions, tokens, page_table, top_k, inv_temperature, count_input=None,
                        penalties=None, raw_logits=False):
        """A decode step returning each row's sampling candidates
        (q35_runtime_step_candidates): arrays [batch][64] of values and tokens,
        and the raw logits [batch][vocab] when asked."""
        slots = np.ascontiguousarray(slots, np.int32)
        positions = np.ascontiguousarray(positions, np.int32)
        tokens = np.ascontiguousarray(tokens, np.int32)
        b = slots.size
        table = np.ascontiguousarray(page_table, np.int32).reshape(b, -1)
        ci = np.ascontiguousarray(count_input if count_input is not None else np.zeros(b), np.uint8)
        pen = np.ascontiguousarray(penalties if penalties is not None else np.ones(b), np.float32)
        d = StepDesc(b, slots.ctypes.data_as(POINTER(c_int32)), positions.ctypes.data_as(POINTER(c_int32)),
                     tokens.ctypes.data_as(POINTER(c_int32)), ci.ctypes.data_as(POINTER(c_uint8)),
                     pen.ctypes.data_as(POINTER(c_float)), table.ctypes.data_as(POINTER(c_int32)), table.shape[1])
        rs = (RowSampling * b)(*[RowSampling(int(k), float(t)) for k, t in zip(
            np.broadcast_to(top_k, b), np.broadcast_to(inv_temperature, b))])
        cand = (Candidate * (b * MAX_CANDIDATES))()
        lg = np.empty((b, self.model.dims.vocab), np.float32) if raw_logits else None
        self.ctx.check(lib.q35_runtime_step_candidates(self.handle, ctypes.byref(d), ctypes.byref(rs),
                                                       ctypes.byref(cand), _ptr(lg)), "step candidates")
        arr = np.frombuffer(cand, dtype=np.dtype([("value", np.float32), ("token", np.int32)])).reshape(
            b, MAX_CANDIDATES).copy()
        return (arr, lg) if raw_logits else arr

    def slot_counts(self, slot):
        out = np.empty(self.model.dims.vocab, np.int32)
        self.ctx.check(lib.q35_slot_counts(self.handle, int(slot), _ptr(out), out.size), "slot counts")
        return out

    def prefill(self, slot, pos0, tokens, page_table, penalty=1.0):
        """Chunked prefill of one request (q35_runtime_prefill): returns the
        greedy token after the chunk's last position."""
        tokens = np.ascontiguousarray(tokens, np.int32)
        table = np.ascontiguousarray(page_table, np.int32).ravel()
        out = np.empty(1, np.int32)
        self.ctx.check(lib.q35_runtime_prefill(self.handle, int(slot), int(pos0), _ptr(tokens), tokens.size,
                                               _ptr(table), table.size, float(penalty), _ptr(out)),
                       "runtime prefill")
        return int(out[0])

    def step_segments(self, segments, sampling=None, raw_logits=False):
        """One packed step (q35_runtime_step_segments). `segments` is a list of
        dicts with slot, pos0, tokens, page_table and optional penalty,
        count_input (0), want_token (1). Greedy: returns the token per segment
        (-1 without want_token). With `sampling` (a (top_k, inv_temperature)
        pair per segment): returns the candidate arrays [segments][64] (and the
        raw logits [segments][vocab] when asked)."""
        n = len(segments)
        keep = []
        arr = (Segment * n)()
        for i, g in enumerate(segments):
            toks = np.ascontiguousarray(g["tokens"], np.int32).ravel()
            table = np.ascontiguousarray(g["page_table"], np.int32).ravel()
            keep += [toks, table]
            arr[i] = Segment(int(g["slot"]), int(g["pos0"]), toks.size, toks.ctypes.data_as(POINTER(c_int32)),
                             table.ctypes.data_as(POINTER(c_int32)), table.size, float(g.get("penalty", 1.0)),
                             int(g.get("count_input", 0)), int(g.get("want_token", 1)))
        out = np.empty(n, np.int32)
        if sampling is None:
            self.ctx.check(lib.q35_runtime_step_segments(self.handle, arr, n, None, _ptr(out), None, None),
                           "step segments")
            return out
        rs = (RowSampling * n)(*[RowSampling(int(k), float(t)) for k, t in sampling])
        cand = (Candidate * (n * MAX_CANDIDATES))()
        lg = np.empty((n, self.model.dims.vocab), np.float32) if raw_logits else None
        self.ctx.check(lib.q35_runtime_step_segments(self.handle, arr, n, rs, _ptr(out), cand, _ptr(lg)),
                       "step segments")
        c = np.frombuffer(cand, dtype=np.dtype([("value", np.float32), ("token", np.int32)])).reshape(
            n, MAX_CANDIDATES).copy()
        return (c, lg) if raw_logits else c

    def head(self, slot, hidden, penalty=1.0):
        """Greedy head of one final normalized hidden row with the slot's
        penalty counts (q35_runtime_head)."""
        hidden = np.ascontiguousarray(hidden, np.float32)
        out = c_int32()
        self.ctx.check(lib.q35_runtime_head(self.handle, int(slot), _ptr(hidden), float(penalty), ctypes.byref(out)),
                       "runtime head")
        return out.value

    def head_candidates(self, slot, hidden, top_k, inv_temperature, penalty=1.0, raw_logits=False):
        """Sampling candidates of one final normalized hidden row
        (q35_runtime_head_candidates): [64] values and tokens, and the raw
        logits [vocab] when asked."""
        hidden = np.ascontiguousarray(hidden, np.float32)
        rs = RowSampling(int(top_k), float(inv_temperature))
        cand = (Candidate * MAX_CANDIDATES)()
        lg = np.empty(self.model.dims.vocab, np.float32) if raw_logits else None
        self.ctx.check(lib.q35_runtime_head_candidates(self.handle, int(slot), _ptr(hidden), float(penalty),
                                                       ctypes.byref(rs), ctypes.byref(cand), _ptr(lg)),
                       "head candidates")
        arr = np.frombuffer(cand, dtype=np.dtype([("value", np.float32), ("token", np.int32)])).copy()
        return (arr, lg) if raw_logits else arr

    def set_fused(self, enable=True):
        """Fused decode projections on or off (q35_runtime_set_fused; both give identical bits)."""
        self.ctx.check(lib.q35_runtime_set_fused(self.handle, int(enable)), "set fused")

    def set_trace(self, enable=True):
        """Stage trace of the next steps (q35_runtime_set_trace, a test hook)."""
        self.ctx.check(lib.q35_runtime_set_trace(self.handle, int(enable)), "set trace")

    def trace(self, layer, point, dtype=np.float32):
        """The traced bytes of (layer, point) of the last step as a flat array
        of `dtype` (None when the step did not trace that point)."""
        n = c_size_t()
        self.ctx.check(lib.q35_runtime_trace_read(self.handle, int(layer), int(point), None, 0, ctypes.byref(n)),
                       "trace size")
        if n.value == 0:
            return None
        out = np.empty(n.value // np.dtype(dtype).itemsize, dtype)
        self.ctx.check(lib.q35_runtime_trace_read(self.handle, int(layer), int(point), _ptr(out), out.nbytes,
                                                  ctypes.byref(n)), "trace read")
        return out

    def _rt(self):
        return self.handle

    def last_hidden(self, batch):
        out = np.empty((batch, self.model.dims.hidden), np.float32)
        self.ctx.check(lib.q35_runtime_last_hidden(self.handle, _ptr(out), out.size), "last hidden")
        return out

    def close(self):
        if self.handle is not None:
            lib.q35_runtime_destroy(self.handle)
            self.handle = None


class Engine(_Profiled):
    """CpuEngine mirror (include/qwen35x/runtime/cpu_engine.h:173-215), greedy requests."""

    def __init__(self, model, max_resident_requests=32, max_context=8192, max_decode_batch_size=32,
                 prefill_chunk_size=128, page_tokens=16, use_graphs=True, max_prefix_bytes=0,
                 max_prefill_requests=1, packed_steps=False, max_queued_requests=0, max_buffered_tokens=256):
        """max_queued_requests > 0 selects serving mode (step / read_output);
        0 the direct mode (advance / advance_batch), as CpuEngineConfig."""
        self.model, self.ctx = model, model.ctx
        cfg = EngineConfig(max_resident_requests, max_context, max_decode_batch_size, prefill_chunk_size,
                           page_tokens, int(use_graphs), max_prefix_bytes, int(max_prefill_requests),
                           int(packed_steps), int(max_queued_requests), int(max_buffered_tokens))
        h = c_void_p()
        self.ctx.check(lib.q35_engine_create(model.handle, ctypes.byref(cfg), ctypes.byref(h)), "engine create")
        self.handle = h

    def _rt(self):
        return lib.q35_engine_runtime(self.handle)

    def _check(self, status, what):
        if status != Q35_OK:
            raise Q35Error(f"{what}: {STATUS.get(status, status)} "
                           f"{lib.q35_engine_last_error(self.handle).decode(errors='replace')}")

    def submit(self, prompt, max_new_tokens=128, repetition_penalty=1.0, stop_token_ids=(), prefix=0):
        prompt = np.ascontiguousarray(prompt, np.int32)
        stops = np.ascontiguousarray(stop_token_ids, np.int32)
        rid = c_uint64()
        self._check(lib.q35_engine_submit_prefixed(self.handle, _ptr(prompt), prompt.size, max_new_tokens,
                                                   repetition_penalty, _ptr(stops) if stops.size else None,
                                                   stops.size, prefix, ctypes.byref(rid)), "submit")
        return rid.value

    def submit_spec(self, prompt, max_new_tokens=128, temperature=0.7, top_p=0.8, top_k=20,
                    repetition_penalty=1.05, seed=-1, stop_token_ids=(), stop_sequences=(), forced_output_tokens=(),
                    logits_callback=None, prefix=0, sampling_constraint=None, selected_logit_tokens=(),
                    selected_logits_callback=None, register_prefix_tokens=0, trust_namespace=None):
        """CpuEngine::submit with a CpuRequestSpec (q35_engine_submit_spec); the
        sampling defaults are SamplingOptions' (options.h:10-13). logits_callback,
        when given, is a Python callable (index, forced_token, logits ndarray) ->
        bool, called with each row's raw logits. sampling_constraint is an object
        with apply(logits ndarray, masked in place) -> bool and accept(token) ->
        bool (CpuSamplingConstraint). selected_logits_callback (same signature as
        logits_callback) receives the logits at selected_logit_tokens."""
        keep = []  # arrays and the callback must outlive the call

        def arr(values, dtype, ctype):
            a = np.ascontiguousarray(values, dtype)
            keep.append(a)
            return a.ctypes.data_as(POINTER(ctype)) if a.size else None, a.size

        prompt_p, n = arr(prompt, np.int32, c_int32)
        stops_p, ns = arr(stop_token_ids, np.int32, c_int32)
        seqs = [np.asarray(q, np.int32) for q in stop_sequences]
        flat_p, _ = arr(np.concatenate(seqs) if seqs else np.zeros(0, np.int32), np.int32, c_int32)
        lens_p, nseq = arr([q.size for q in seqs], np.uintp, c_size_t)
        forced_p, nf = arr(forced_output_tokens, np.int32, c_int32)
        cb = LOGITS_CALLBACK()
        if logits_callback is not None:
            def trampoline(_ctx, index, forced, logits, count):
                try:
                    return 1 if logits_callback(index, forced, np.ctypeslib.as_array(logits, (count,)).copy()) else 0
                except Exception:  # a raising callback fails the request, as returning false does
                    return 0
            cb = LOGITS_CALLBACK(trampoline)
            self._callbacks = getattr(self, "_callbacks", []) + [cb]
        def wrap(fn):
            def trampoline(_ctx, index, forced, logits, count):
                try:
                    return 1 if fn(index, forced, np.ctypeslib.as_array(logits, (count,)).copy()) else 0
                except Exception:  # a raising callback fails the request, as returning false does
                    return 0
            return LOGITS_CALLBACK(trampoline)

        scb = wrap(selected_logits_callback) if selected_logits_callback is not None else LOGITS_CALLBACK()
        sel_p, nsel = arr(selected_logit_tokens, np.int32, c_int32)
        cons = None
        if sampling_constraint is not None:
            def apply(_ctx, logits, count):
                try:
                    return 1 if sampling_constraint.apply(np.ctypeslib.as_array(logits, (count,))) else 0
                except Exception:
                    return 0

            def accept(_ctx, token):
                try:
                    return 1 if sampling_constraint.accept(int(token)) else 0
                except Exception:
                    return 0
            cons = SamplingConstraint(None, CONSTRAINT_APPLY(apply), CONSTRAINT_ACCEPT(accept))
        self._callbacks = getattr(self, "_callbacks", []) + [scb, cons]
        spec = RequestSpec(prompt_p, n, max_new_tokens, temperature, top_p, top_k, repetition_penalty, seed,
                           stops_p, ns, flat_p, lens_p, nseq, forced_p, nf, cb, None, prefix,
                           ctypes.cast(ctypes.pointer(cons), c_void_p) if cons is not None else None,
                           sel_p, nsel, scb, None, int(register_prefix_tokens),
                           trust_namespace.encode() if trust_namespace is not None else None)
        rid = c_uint64()
        self._check(lib.q35_engine_submit_spec(self.handle, ctypes.byref(spec), ctypes.byref(rid)), "submit")
        return rid.value

    def register_prefix(self, tokens, trust_namespace):
        """CpuEngine::register_prefix: a pinned prefix handle (release_prefix unpins)."""
        tokens = np.ascontiguousarray(tokens, np.int32)
        h = c_uint64()
        self._check(lib.q35_engine_register_prefix(self.handle, _ptr(tokens), tokens.size,
                                                   trust_namespace.encode(), ctypes.byref(h)), "register_prefix")
        return h.value

    def find_prefix(self, tokens, trust_namespace):
        """CpuEngine::find_prefix: (handle, token count) of the longest cached match, (0, 0) if none."""
        tokens = np.ascontiguousarray(tokens, np.int32)
        h, n = c_uint64(), c_size_t()
        self._check(lib.q35_engine_find_prefix(self.handle, _ptr(tokens), tokens.size, trust_namespace.encode(),
                                               ctypes.byref(h), ctypes.byref(n)), "find_prefix")
        return h.value, n.value

    def release_prefix(self, handle):
        self._check(lib.q35_engine_release_prefix(self.handle, handle), "release_prefix")

    def free_pages(self):
        """Free pages of the engine's KV pool (q35_runtime_free_pages)."""
        return lib.q35_runtime_free_pages(self._rt())

    def stats(self):
        """Engine counters (q35_engine_get_stats) as a dict."""
        st = EngineStats()
        self._check(lib.q35_engine_get_stats(self.handle, ctypes.byref(st)), "stats")
        return {f: getattr(st, f) for f, _ in st._fields_}

    def prefix_stats(self):
        st = PrefixStats()
        self._check(lib.q35_engine_prefix_stats(self.handle, ctypes.byref(st)), "prefix_stats")
        return {f: getattr(st, f) for f, _ in st._fields_}

    def advance(self, rid):
        self._check(lib.q35_engine_advance(self.handle, rid), "advance")

    def advance_batch(self, ids):
        a = np.ascontiguousarray(ids, np.uint64)
        self._check(lib.q35_engine_advance_batch(self.handle, _ptr(a), a.size), "advance_batch")

    def prefill_batch(self, ids):
        a = np.ascontiguousarray(ids, np.uint64)
        self._check(lib.q35_engine_prefill_batch(self.handle, _ptr(a), a.size), "prefill_batch")

    def step(self):
        p = c_int32()
        self._check(lib.q35_engine_step(self.handle, ctypes.byref(p)), "step")
        return bool(p.value)

    def read_output(self, rid, max_tokens=1 << 20):
        """CpuEngine::read_output: up to max_tokens confirmed, unread output
        tokens (serving mode)."""
        out = np.empty(max(int(max_tokens), 1), np.int32)
        n = c_size_t()
        self._check(lib.q35_engine_read_output(self.handle, rid, int(max_tokens), _ptr(out), ctypes.byref(n)),
                    "read_output")
        return out[:n.value].copy()

    def result(self, rid):
        r = RequestResult()
        n = c_size_t()
        self._check(lib.q35_engine_result(self.handle, rid, ctypes.byref(r), None, 0, ctypes.byref(n)), "result")
        toks = np.empty(n.value, np.int32)
        if n.value:
            self._check(lib.q35_engine_result(self.handle, rid, None, _ptr(toks), n.value, None), "result")
        return r, toks

    def terminal(self, rid):
        """Whether the request is complete, cancelled or failed."""
        return REQ_STATUS[self.result(rid)[0].status] in ("complete", "cancelled", "failed")

    def cancel(self, rid):
        self._check(lib.q35_engine_cancel(self.handle, rid), "cancel")

    def release(self, rid):
        self._check(lib.q35_engine_release(self.handle, rid), "release")

    def close(self):
        if self.handle is not None:
            lib.q35_engine_destroy(self.handle)
            self.handle = None
