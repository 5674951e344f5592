"""Python host-side mirror of the qm38 C ABI (include/qm38.h).

The class and method names follow the reference runtime
(/root/reference/src/metal_runtime.rs, `MetalRuntime`): `q4_affine_matvec_batch`
<-> q4_affine_matvec_mapped_batch, `gqa_attention_q8` <-> gqa_attention_q8,
`deltanet_step` <-> deltanet_step, and so on.  Errors raise `QmError`, whose
`status` names the reference's `MetalRuntimeError` variant equivalent.

Activations are passed as device tensors (torch is used only to own HBM and
the stream); every computation runs in libqm38.so.  There is no fallback: if
the library is missing, `load()` raises.
"""
from __future__ import annotations

import ctypes as C
import weakref
import os
from pathlib import Path

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "libqm38.so"

QM_STATUS = [
    "QM_OK", "QM_ERR_NO_DEVICE", "QM_ERR_EMPTY_DIMENSION", "QM_ERR_INPUT_NOT_GROUPED",
    "QM_ERR_WRONG_LENGTH", "QM_ERR_INVALID_DELTANET_CONFIG", "QM_ERR_INVALID_ATTENTION_SHAPE",
    "QM_ERR_INVALID_SEQUENCE_LENGTH", "QM_ERR_INVALID_BUFFER_OFFSET",
    "QM_ERR_MAPPED_TENSOR_OUT_OF_RANGE", "QM_ERR_DIMENSION_OVERFLOW", "QM_ERR_COMMAND_FAILED",
    "QM_ERR_ZERO_CAPACITY", "QM_ERR_EMPTY_APPEND", "QM_ERR_CAPACITY_EXCEEDED",
    "QM_ERR_NULL_POINTER", "QM_ERR_OUT_OF_MEMORY", "QM_ERR_MISALIGNED", "QM_ERR_INVALID_ARGUMENT",
    "QM_ERR_INVALID_SNAPSHOT", "QM_ERR_INVALID_SNAPSHOT_ROW", "QM_ERR_MODEL_FORMAT", "QM_ERR_INVALID_TENSOR",
    "QM_ERR_GRAPH_STALE",
]

# Every symbol include/qm38.h declares (checked by tests/test_abi.py).
EXPORTS = [
    "qm_status_string", "qm_last_error_message",
    "qm_runtime_create", "qm_runtime_destroy", "qm_runtime_set_stream", "qm_runtime_synchronize",
    "qm_device_alloc", "qm_device_free", "qm_upload", "qm_copy_to_device", "qm_copy_to_host",
    "qm_q4_project", "qm_q4_project_set", "qm_q4_swiglu", "qm_q4_mlp", "qm_q4_argmax", "qm_q4_job_from_mapped",
    "qm_kv_create", "qm_kv_destroy", "qm_kv_length", "qm_kv_capacity", "qm_kv_allocated_pages", "qm_kv_page_for_token",
    "qm_kv_reserve", "qm_kv_truncate", "qm_kv_clone", "qm_kv_read",
    "qm_attn_decode", "qm_attn_decode_noalloc", "qm_attn_prefill", "qm_attn_prepare",
    "qm_dn_weights_create", "qm_dn_weights_destroy", "qm_dn_state_create", "qm_dn_state_destroy",
    "qm_dn_state_clone", "qm_dn_state_read", "qm_dn_state_write", "qm_dn_step", "qm_dn_prefill",
    "qm_dn_snapshots_create", "qm_dn_snapshots_destroy", "qm_dn_prefill_snapshots", "qm_dn_snapshot_restore",
    "qm_store_open", "qm_store_close", "qm_store_tensor_count", "qm_store_tensor_info", "qm_store_upload",
    "qm_store_upload_q4",
    "qm_residual_rmsnorm", "qm_residual_add", "qm_decode_state_create", "qm_decode_state_destroy",
    "qm_decode_state_hidden", "qm_decode_layers", "qm_decode_graph_create", "qm_decode_graph_run",
    "qm_decode_graph_destroy",
]


class QmError(RuntimeError):
    def __init__(self, status: int, message: str):
        self.status = QM_STATUS[status] if 0 <= status < len(QM_STATUS) else f"status {status}"
        self.code = status
        super().__init__(message)


class Q4Job(C.Structure):
    _fields_ = [("weights", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p),
                ("out_rows", C.c_uint32)]


class Buffer(C.Structure):
    """qm_buffer: a device allocation and its length in bytes."""
    _fields_ = [("base", C.c_void_p), ("length", C.c_uint64)]


class Q4MappedJob(C.Structure):
    """qm_q4_mapped_job (MappedQ4AffineJob, metal_runtime.rs:155-192)."""
    _fields_ = [("weights", Buffer), ("weight_offset", C.c_uint64), ("scales", Buffer),
                ("scale_offset", C.c_uint64), ("biases", Buffer), ("bias_offset", C.c_uint64),
                ("out_rows", C.c_uint32)]


class DnConfig(C.Structure):
    _fields_ = [("key_heads", C.c_uint32), ("value_heads", C.c_uint32), ("key_head_dim", C.c_uint32),
                ("value_head_dim", C.c_uint32), ("conv_kernel_size", C.c_uint32)]


class Q4Matrix(C.Structure):
    """qm_q4_matrix: a Q4 matrix uploaded from a weight store."""
    _fields_ = [("weights", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p),
                ("out_rows", C.c_uint32), ("in_elems", C.c_uint32)]


class RopeConfig(C.Structure):
    """qm_rope_config (RopeParameters, native.rs:119-197)."""
    _fields_ = [("head_dim", C.c_uint32), ("rotary_dim", C.c_uint32), ("rope_theta", C.c_float),
                ("mrope_section1", C.c_uint32), ("mrope_section2", C.c_uint32), ("has_mrope_sections", C.c_uint32)]


class DecodeLinearLayer(C.Structure):
    """qm_decode_linear_layer (MetalDecodeLinearLayer, metal_runtime.rs:304-318)."""
    _fields_ = [("input_norm", C.c_void_p), ("post_attention_norm", C.c_void_p),
                ("qkv", Q4Job), ("z", Q4Job), ("b", Q4Job), ("a", Q4Job), ("out_proj", Q4Job),
                ("dn_weights", C.c_void_p), ("dn_state", C.c_void_p),
                ("gate", Q4Job), ("up", Q4Job), ("down", Q4Job)]


class DecodeFullLayer(C.Structure):
    """qm_decode_full_layer (MetalDecodeFullLayer, metal_runtime.rs:385-399)."""
    _fields_ = [("input_norm", C.c_void_p), ("post_attention_norm", C.c_void_p),
                ("q_proj", Q4Job), ("k_proj", Q4Job), ("v_proj", Q4Job), ("o_proj", Q4Job),
                ("q_norm", C.c_void_p), ("k_norm", C.c_void_p), ("num_heads", C.c_uint32),
                ("rope", RopeConfig), ("kv", C.c_void_p),
                ("gate", Q4Job), ("up", Q4Job), ("down", Q4Job)]


class DecodeLayer(C.Structure):
    _fields_ = [("linear", C.POINTER(DecodeLinearLayer)), ("full", C.POINTER(DecodeFullLayer))]


_lib = None


def load(path: str | os.PathLike | None = None) -> C.CDLL:
    """Loads libqm38.so (raises if it has not been built)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(f"{p} is missing: run `python qwen38-metal_amd/build.py`")
    # One HIP runtime per process: torch ships its own libamdhip64 (same
    # SONAME as /opt/rocm's).  Loading torch first makes libqm38 bind to the
    # runtime that owns the tensors and streams handed to it; loading libqm38
    # first would bring in a second HIP runtime that cannot share the device.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = C.CDLL(str(p))
    vp, u32, i32 = C.c_void_p, C.c_uint32, C.c_int
    sig = {
        "qm_status_string": ([i32], C.c_char_p),
        "qm_last_error_message": ([], C.c_char_p),
        "qm_runtime_create": ([i32, C.POINTER(vp)], i32),
        "qm_runtime_destroy": ([vp], None),
        "qm_runtime_set_stream": ([vp, vp], i32),
        "qm_runtime_synchronize": ([vp], i32),
        "qm_device_alloc": ([vp, C.c_size_t, C.POINTER(vp)], i32),
        "qm_device_free": ([vp, vp], i32),
        "qm_upload": ([vp, vp, C.c_size_t, C.POINTER(vp)], i32),
        "qm_copy_to_device": ([vp, vp, vp, C.c_size_t], i32),
        "qm_copy_to_host": ([vp, vp, vp, C.c_size_t], i32),
        "qm_q4_project": ([vp, C.POINTER(Q4Job), i32, vp, u32, u32, C.POINTER(vp)], i32),
        "qm_q4_swiglu": ([vp, C.POINTER(Q4Job), C.POINTER(Q4Job), vp, u32, u32, vp], i32),
        "qm_q4_mlp": ([vp, C.POINTER(Q4Job), C.POINTER(Q4Job), C.POINTER(Q4Job), vp, u32, u32, vp], i32),
        "qm_q4_project_set": ([vp, C.POINTER(Q4Job), C.POINTER(C.POINTER(Q4Job)), i32, vp, u32, u32,
                               C.POINTER(vp)], i32),
        "qm_q4_argmax": ([vp, C.POINTER(Q4Job), vp, u32, u32, vp], i32),
        "qm_q4_job_from_mapped": ([C.POINTER(Q4MappedJob), u32, C.POINTER(Q4Job)], i32),
        "qm_kv_create": ([vp, u32, u32, u32, u32, C.POINTER(vp)], i32),
        "qm_kv_destroy": ([vp], None),
        "qm_kv_length": ([vp], u32),
        "qm_kv_capacity": ([vp], u32),
        "qm_kv_allocated_pages": ([vp], u32),
        "qm_kv_page_for_token": ([vp, u32], C.c_int64),
        "qm_kv_reserve": ([vp, u32], i32),
        "qm_kv_truncate": ([vp, u32], i32),
        "qm_kv_clone": ([vp, C.POINTER(vp)], i32),
        "qm_kv_read": ([vp, vp, vp, vp, vp], i32),
        "qm_attn_decode": ([vp, C.POINTER(vp), u32, vp, vp, vp, vp, u32, vp], i32),
        "qm_attn_decode_noalloc": ([vp, C.POINTER(vp), u32, vp, vp, vp, vp, u32, vp], i32),
        "qm_attn_prefill": ([vp, vp, vp, vp, vp, vp, u32, u32, vp], i32),
        "qm_attn_prepare": ([vp, C.POINTER(RopeConfig), u32, u32, u32, vp, vp, vp, vp, C.c_float, vp, u32, vp, vp,
                             vp], i32),
        "qm_dn_weights_create": ([vp, C.POINTER(DnConfig), vp, vp, vp, vp, C.POINTER(vp)], i32),
        "qm_dn_weights_destroy": ([vp], None),
        "qm_dn_state_create": ([vp, vp, C.POINTER(vp)], i32),
        "qm_dn_state_destroy": ([vp], None),
        "qm_dn_state_clone": ([vp, C.POINTER(vp)], i32),
        "qm_dn_state_read": ([vp, vp, vp], i32),
        "qm_dn_state_write": ([vp, vp, vp], i32),
        "qm_dn_step": ([vp, vp, vp, vp, vp, vp, vp, C.c_float, vp], i32),
        "qm_dn_prefill": ([vp, vp, vp, vp, vp, vp, vp, vp, u32, C.c_float, vp], i32),
        "qm_store_open": ([C.c_char_p, C.POINTER(vp)], i32),
        "qm_store_close": ([vp], None),
        "qm_store_tensor_count": ([vp], u32),
        "qm_store_tensor_info": ([vp, C.c_char_p, C.c_char_p, C.c_size_t, C.POINTER(u32), C.POINTER(C.c_uint64),
                                  u32, C.POINTER(C.c_uint64)], i32),
        "qm_store_upload": ([vp, vp, C.c_char_p, C.POINTER(vp), C.POINTER(C.c_uint64)], i32),
        "qm_store_upload_q4": ([vp, vp, C.c_char_p, C.POINTER(Q4Matrix)], i32),
        "qm_dn_snapshots_create": ([vp, vp, u32, C.POINTER(vp)], i32),
        "qm_dn_snapshots_destroy": ([vp], None),
        "qm_dn_prefill_snapshots": ([vp, vp, vp, vp, vp, vp, vp, vp, vp, u32, C.c_float, vp], i32),
        "qm_dn_snapshot_restore": ([vp, u32, vp], i32),
        "qm_residual_rmsnorm": ([vp, vp, vp, vp, u32, u32, C.c_float, vp], i32),
        "qm_residual_add": ([vp, vp, vp, C.c_size_t], i32),
        "qm_decode_state_create": ([vp, u32, C.POINTER(vp)], i32),
        "qm_decode_state_destroy": ([vp], None),
        "qm_decode_state_hidden": ([vp], vp),
        "qm_decode_layers": ([vp, vp, C.POINTER(DecodeLayer), u32, C.POINTER(u32), C.c_float], i32),
        "qm_decode_graph_create": ([vp, vp, C.POINTER(DecodeLayer), u32, C.c_float, C.POINTER(vp)], i32),
        "qm_decode_graph_run": ([vp, C.POINTER(u32)], i32),
        "qm_decode_graph_destroy": ([vp], None),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    if path is None:
        _lib = lib
    return lib


def _check(status: int) -> None:
    if status != 0:
        msg = load().qm_last_error_message().decode()
        raise QmError(status, msg)


def _ptr(t) -> int | None:
    """Device address of a torch tensor / raw int, or None."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


class Runtime:
    """One runtime per HIP device (MetalRuntime::new, metal_runtime.rs:641)."""

    def __init__(self, device: int = 0):
        self.lib = load()
        h = C.c_void_p()
        _check(self.lib.qm_runtime_create(device, C.byref(h)))
        self.handle = h
        self.device = device
        # Objects created on this runtime; closed before it (they use its stream).
        self._children = weakref.WeakSet()

    def close(self) -> None:
        if self.handle:
            for child in list(self._children):
                child.close()
            self.lib.qm_runtime_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_stream(self, stream) -> None:
        """stream: a torch.cuda.Stream, a raw hipStream_t int, or None."""
        raw = getattr(stream, "cuda_stream", stream)
        _check(self.lib.qm_runtime_set_stream(self.handle, raw))

    def synchronize(self) -> None:
        _check(self.lib.qm_runtime_synchronize(self.handle))

    def device_buffer(self, data=None, nbytes: int | None = None) -> "DeviceBuffer":
        """A library allocation (qm_device_alloc) of nbytes, or holding a copy of
        the numpy array `data` (qm_upload)."""
        p = C.c_void_p()
        if data is not None:
            import numpy as np
            a = np.ascontiguousarray(data)
            _check(self.lib.qm_upload(self.handle, a.ctypes.data, a.nbytes, C.byref(p)))
            return DeviceBuffer(self, p.value, a.nbytes)
        _check(self.lib.qm_device_alloc(self.handle, nbytes, C.byref(p)))
        return DeviceBuffer(self, p.value, nbytes)

    # ---- Q4 projections --------------------------------------------------
    @staticmethod
    def job(weights, scales, biases, out_rows: int) -> Q4Job:
        j = Q4Job(_ptr(weights), _ptr(scales), _ptr(biases), out_rows)
        j._refs = (weights, scales, biases)  # keep device tensors alive while the job exists
        return j

    def q4_project(self, jobs, x, in_elems: int, M: int, outputs) -> None:
        arr = (Q4Job * len(jobs))(*jobs)
        outs = (C.c_void_p * len(outputs))(*[_ptr(o) for o in outputs])
        _check(self.lib.qm_q4_project(self.handle, arr, len(jobs), _ptr(x), in_elems, M, outs))

    def q4_project_set(self, jobs, ups, x, in_elems: int, M: int, outputs) -> None:
        """jobs[j] plain (ups[j] None) or the gate of a SwiGLU pair with up ups[j]."""
        arr = (Q4Job * len(jobs))(*jobs)
        upp = (C.POINTER(Q4Job) * len(jobs))(*[C.pointer(u) if u is not None else None for u in ups])
        outs = (C.c_void_p * len(outputs))(*[_ptr(o) for o in outputs])
        _check(self.lib.qm_q4_project_set(self.handle, arr, upp, len(jobs), _ptr(x), in_elems, M, outs))

    def q4_swiglu(self, gate: Q4Job, up: Q4Job, x, in_elems: int, M: int, h) -> None:
        _check(self.lib.qm_q4_swiglu(self.handle, C.byref(gate), C.byref(up), _ptr(x), in_elems, M, _ptr(h)))

    def q4_mlp(self, gate: Q4Job, up: Q4Job, down: Q4Job, x, in_elems: int, M: int, y) -> None:
        _check(self.lib.qm_q4_mlp(self.handle, C.byref(gate), C.byref(up), C.byref(down), _ptr(x),
                                  in_elems, M, _ptr(y)))

    def q4_affine_argmax(self, job: Q4Job, x, in_elems: int, M: int, ids) -> None:
        """ids (uint32/int32 [M], device) = per-row argmax of job(x) (q4_affine_argmax_mapped_batch)."""
        _check(self.lib.qm_q4_argmax(self.handle, C.byref(job), _ptr(x), in_elems, M, _ptr(ids)))

    @staticmethod
    def mapped_job(weights, weight_offset: int, scales, scale_offset: int, biases, bias_offset: int,
                   out_rows: int, in_elems: int) -> Q4Job:
        """A Q4Job from (buffer, offset) tensors, each buffer a (base, length) pair
        (MappedQ4AffineJob::new + validate_mapped_q4_affine_shape)."""
        m = Q4MappedJob(Buffer(*weights), weight_offset, Buffer(*scales), scale_offset, Buffer(*biases),
                        bias_offset, out_rows)
        j = Q4Job()
        _check(load().qm_q4_job_from_mapped(C.byref(m), in_elems, C.byref(j)))
        return j

    # ---- Q8 KV + attention -------------------------------------------------
    def create_q8_kv_state(self, kv_heads: int, head_dim: int, max_tokens: int = 0,
                           page_tokens: int = 16) -> "KvCache":
        """create_q8_kv_state; max_tokens = 0 grows without limit (the reference's policy)."""
        return KvCache(self, kv_heads, head_dim, page_tokens, max_tokens)

    def gqa_attention_q8(self, seqs, q, gate, k, v, num_heads: int, o) -> None:
        arr = (C.c_void_p * len(seqs))(*[s.handle for s in seqs])
        _check(self.lib.qm_attn_decode(self.handle, arr, len(seqs), _ptr(q), _ptr(gate), _ptr(k), _ptr(v),
                                       num_heads, _ptr(o)))

    def gqa_attention_q8_noalloc(self, seqs, q, gate, k, v, num_heads: int, o) -> None:
        """qm_attn_decode_noalloc: no device allocation (caches must have room)."""
        arr = (C.c_void_p * len(seqs))(*[s.handle for s in seqs])
        _check(self.lib.qm_attn_decode_noalloc(self.handle, arr, len(seqs), _ptr(q), _ptr(gate), _ptr(k), _ptr(v),
                                               num_heads, _ptr(o)))

    def gqa_attention_q8_prefill(self, seq, q, gate, k, v, num_heads: int, rows: int, o) -> None:
        _check(self.lib.qm_attn_prefill(self.handle, seq.handle, _ptr(q), _ptr(gate), _ptr(k), _ptr(v),
                                        num_heads, rows, _ptr(o)))

    def attn_prepare(self, rope: RopeConfig, rows: int, num_heads: int, kv_heads: int, q_with_gate, k, q_norm,
                     k_norm, epsilon: float, q_out, gate_out, k_out, positions=None, position_base: int = 0) -> None:
        """Full-attention q/k preparation (qm_attn_prepare): RMSNorm, (M-)RoPE
        and the query/gate split of qwen38_gqa_prepare_query/_key."""
        _check(self.lib.qm_attn_prepare(self.handle, C.byref(rope), rows, num_heads, kv_heads, _ptr(q_with_gate),
                                        _ptr(k), _ptr(q_norm), _ptr(k_norm), epsilon, _ptr(positions),
                                        position_base, _ptr(q_out), _ptr(gate_out), _ptr(k_out)))

    # ---- DeltaNet ---------------------------------------------------------
    def create_deltanet_weights(self, config: DnConfig, conv_weight, a_log, dt_bias, norm) -> "DnWeights":
        return DnWeights(self, config, conv_weight, a_log, dt_bias, norm)

    def deltanet_step(self, weights, state, qkv, z, b, a, epsilon: float, out) -> None:
        _check(self.lib.qm_dn_step(self.handle, weights.handle, state.handle, _ptr(qkv), _ptr(z), _ptr(b),
                                   _ptr(a), epsilon, _ptr(out)))

    def deltanet_prefill_with_snapshots(self, weights, source, state, snapshots, qkv, z, b, a, rows: int,
                                        epsilon: float, out) -> None:
        """deltanet_prefill_from_with_snapshots: also records the state after
        each of the first rows - 1 rows into `snapshots`."""
        _check(self.lib.qm_dn_prefill_snapshots(self.handle, weights.handle, source.handle if source else None,
                                                state.handle, snapshots.handle, _ptr(qkv), _ptr(z), _ptr(b),
                                                _ptr(a), rows, epsilon, _ptr(out)))

    def deltanet_prefill(self, weights, state, qkv, z, b, a, rows: int, epsilon: float, out,
                         source=None) -> None:
        src = source.handle if source is not None else None
        _check(self.lib.qm_dn_prefill(self.handle, weights.handle, src, state.handle, _ptr(qkv), _ptr(z),
                                      _ptr(b), _ptr(a), rows, epsilon, _ptr(out)))


    # ---- residual stream and decode graph ----------------------------------
    def residual_rmsnorm(self, hidden, delta, weights, rows: int, elements: int, epsilon: float, out) -> None:
        """hidden += delta (when given), out = bf16(rms_norm(hidden) * weights)
        (qwen38_add_in_place + qwen38_rms_norm(_rows))."""
        _check(self.lib.qm_residual_rmsnorm(self.handle, _ptr(hidden), _ptr(delta), _ptr(weights), rows, elements,
                                            epsilon, _ptr(out)))

    def residual_add(self, hidden, delta, count: int) -> None:
        _check(self.lib.qm_residual_add(self.handle, _ptr(hidden), _ptr(delta), count))

    def create_decode_state(self, hidden_elements: int) -> "DecodeState":
        return DecodeState(self, hidden_elements)

    def decode_layers(self, state: "DecodeState", layers, position, epsilon: float) -> None:
        """One token through `layers` (decode_layers, metal_runtime.rs:2022)."""
        arr, _keep = _layer_array(layers)
        pos = (C.c_uint32 * 3)(*_position3(position))
        _check(self.lib.qm_decode_layers(self.handle, state.handle, arr, len(layers), pos, epsilon))


def _position3(position):
    if isinstance(position, int):
        return (position, position, position)
    p = tuple(int(v) for v in position)
    assert len(p) == 3
    return p


def _layer_array(layers):
    """DecodeLinearLayer / DecodeFullLayer list -> qm_decode_layer array (and the
    objects it points at, which must stay alive for the call)."""
    arr = (DecodeLayer * len(layers))()
    for i, L in enumerate(layers):
        if isinstance(L, DecodeLinearLayer):
            arr[i].linear = C.pointer(L)
        elif isinstance(L, DecodeFullLayer):
            arr[i].full = C.pointer(L)
        else:
            raise TypeError(f"layer {i}: {type(L).__name__}")
    return arr, list(layers)


class DecodeState:
    """qm_decode_state: the fp32 residual row of one decoding request and its
    intermediates (MetalDecodeState, metal_runtime.rs:246)."""

    def __init__(self, rt: Runtime, hidden_elements: int):
        self.rt = rt
        self.hidden_elements = hidden_elements
        h = C.c_void_p()
        _check(rt.lib.qm_decode_state_create(rt.handle, hidden_elements, C.byref(h)))
        self.handle = h
        rt._children.add(self)

    @property
    def hidden_ptr(self) -> int:
        return self.rt.lib.qm_decode_state_hidden(self.handle)

    def close(self) -> None:
        if self.handle:
            self.rt.lib.qm_decode_state_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DecodeGraph:
    """qm_decode_graph: one token's launches captured as HIP graph segments."""

    def __init__(self, rt: Runtime, state: DecodeState, layers, epsilon: float):
        self.rt = rt
        arr, self._keep = _layer_array(layers)
        h = C.c_void_p()
        _check(rt.lib.qm_decode_graph_create(rt.handle, state.handle, arr, len(layers), epsilon, C.byref(h)))
        self.handle = h
        rt._children.add(self)

    def run(self, position) -> None:
        pos = (C.c_uint32 * 3)(*_position3(position))
        _check(self.rt.lib.qm_decode_graph_run(self.handle, pos))

    def close(self) -> None:
        if self.handle:
            self.rt.lib.qm_decode_graph_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class KvCache:
    """Paged Q8 KV cache (Q8KvState + LogicalPageTable)."""

    def __init__(self, rt: Runtime, kv_heads: int, head_dim: int, page_tokens: int, max_tokens: int,
                 handle=None):
        self.rt = rt
        self.kv_heads = kv_heads
        self.head_dim = head_dim
        if handle is None:
            h = C.c_void_p()
            _check(rt.lib.qm_kv_create(rt.handle, kv_heads, head_dim, page_tokens, max_tokens, C.byref(h)))
            handle = h
        self.handle = handle
        rt._children.add(self)

    def close(self) -> None:
        if self.handle:
            self.rt.lib.qm_kv_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def sequence_length(self) -> int:
        return self.rt.lib.qm_kv_length(self.handle)

    @property
    def capacity_tokens(self) -> int:
        return self.rt.lib.qm_kv_capacity(self.handle)

    @property
    def allocated_pages(self) -> int:
        return self.rt.lib.qm_kv_allocated_pages(self.handle)

    def page_for_token(self, token: int):
        r = self.rt.lib.qm_kv_page_for_token(self.handle, token)
        return None if r < 0 else r

    def reserve(self, additional: int) -> None:
        _check(self.rt.lib.qm_kv_reserve(self.handle, additional))

    def truncate(self, length: int) -> None:
        _check(self.rt.lib.qm_kv_truncate(self.handle, length))

    def clone(self) -> "KvCache":
        h = C.c_void_p()
        _check(self.rt.lib.qm_kv_clone(self.handle, C.byref(h)))
        return KvCache(self.rt, self.kv_heads, self.head_dim, 16, 0, handle=h)

    def read(self):
        """Returns (keys int8 [T][KVH][d], values, key_scales f32 [T][KVH], value_scales)."""
        import numpy as np
        T = self.sequence_length
        keys = np.zeros((T, self.kv_heads, self.head_dim), np.int8)
        values = np.zeros_like(keys)
        ks = np.zeros((T, self.kv_heads), np.float32)
        vs = np.zeros_like(ks)
        _check(self.rt.lib.qm_kv_read(self.handle, keys.ctypes.data, values.ctypes.data, ks.ctypes.data,
                                      vs.ctypes.data))
        return keys, values, ks, vs


class DnWeights:
    def __init__(self, rt: Runtime, config: DnConfig, conv_weight, a_log, dt_bias, norm):
        import numpy as np
        self.rt = rt
        self.config = config
        arrs = [np.ascontiguousarray(a, dtype=np.float32) for a in (conv_weight, a_log, dt_bias, norm)]
        h = C.c_void_p()
        _check(rt.lib.qm_dn_weights_create(rt.handle, C.byref(config), *[a.ctypes.data for a in arrs],
                                           C.byref(h)))
        self.handle = h
        rt._children.add(self)

    def close(self) -> None:
        if self.handle:
            self.rt.lib.qm_dn_weights_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def create_snapshots(self, rows: int) -> "DnSnapshots":
        """create_deltanet_snapshots: room for `rows` verification state images."""
        h = C.c_void_p()
        _check(self.rt.lib.qm_dn_snapshots_create(self.rt.handle, self.handle, rows, C.byref(h)))
        return DnSnapshots(self, h, rows)

    def create_state(self) -> "DnState":
        h = C.c_void_p()
        _check(self.rt.lib.qm_dn_state_create(self.rt.handle, self.handle, C.byref(h)))
        return DnState(self, h)


class DnState:
    def __init__(self, weights: DnWeights, handle):
        self.weights = weights
        self.rt = weights.rt
        self.handle = handle
        self.rt._children.add(self)

    def close(self) -> None:
        if self.handle:
            self.rt.lib.qm_dn_state_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def clone(self) -> "DnState":
        h = C.c_void_p()
        _check(self.rt.lib.qm_dn_state_clone(self.handle, C.byref(h)))
        return DnState(self.weights, h)

    def _shapes(self):
        c = self.weights.config
        channels = 2 * c.key_heads * c.key_head_dim + c.value_heads * c.value_head_dim
        return (channels, max(c.conv_kernel_size - 1, 0)), (c.value_heads, c.value_head_dim, c.key_head_dim)

    def read(self):
        import numpy as np
        hs, ss = self._shapes()
        hist = np.zeros(hs, np.float32)
        rec = np.zeros(ss, np.float32)
        _check(self.rt.lib.qm_dn_state_read(self.handle, hist.ctypes.data if hist.size else None,
                                            rec.ctypes.data))
        return hist, rec

    def write(self, hist, rec) -> None:
        import numpy as np
        hist = None if hist is None else np.ascontiguousarray(hist, np.float32)
        rec = None if rec is None else np.ascontiguousarray(rec, np.float32)
        _check(self.rt.lib.qm_dn_state_write(self.handle, hist.ctypes.data if hist is not None and hist.size else None,
                                             rec.ctypes.data if rec is not None else None))


class DnSnapshots:
    """MetalDeltaNetSnapshots: verification state images."""

    def __init__(self, weights: DnWeights, handle, rows: int):
        self.weights = weights
        self.rt = weights.rt
        self.handle = handle
        self.rows = rows
        self.rt._children.add(self)

    def restore(self, row: int, state: DnState) -> None:
        """restore_deltanet_snapshot: `state` becomes the state after row `row`."""
        _check(self.rt.lib.qm_dn_snapshot_restore(self.handle, row, state.handle))

    def close(self) -> None:
        if self.handle:
            self.rt.lib.qm_dn_snapshots_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class WeightStore:
    """MLX safetensors model directory (qm_store_open; open_mlx_safetensors_dir,
    model.rs:136-197).  Host-only until a tensor is uploaded."""

    def __init__(self, directory, lib=None):
        self.lib = lib or load()
        h = C.c_void_p()
        _check(self.lib.qm_store_open(os.fsencode(directory), C.byref(h)))
        self.handle = h

    def __len__(self) -> int:
        return int(self.lib.qm_store_tensor_count(self.handle))

    def info(self, name: str):
        """(dtype, shape, bytes) of one tensor."""
        dt = C.create_string_buffer(16)
        nd = C.c_uint32()
        shape = (C.c_uint64 * 8)()
        nbytes = C.c_uint64()
        _check(self.lib.qm_store_tensor_info(self.handle, name.encode(), dt, 16, C.byref(nd), shape, 8,
                                             C.byref(nbytes)))
        return dt.value.decode(), tuple(int(shape[i]) for i in range(nd.value)), int(nbytes.value)

    def upload(self, rt: "Runtime", name: str) -> "DeviceBuffer":
        p = C.c_void_p()
        n = C.c_uint64()
        _check(self.lib.qm_store_upload(rt.handle, self.handle, name.encode(), C.byref(p), C.byref(n)))
        return DeviceBuffer(rt, p.value, int(n.value))

    def upload_q4(self, rt: "Runtime", weight_name: str) -> Q4Job:
        """Validated Q4 upload (Q4AffineMatrix::from_store); returns a job whose
        device buffers live as long as it does."""
        m = Q4Matrix()
        _check(self.lib.qm_store_upload_q4(rt.handle, self.handle, weight_name.encode(), C.byref(m)))
        bufs = tuple(DeviceBuffer(rt, p, 0) for p in (m.weights, m.scales, m.biases))
        j = Q4Job(m.weights, m.scales, m.biases, m.out_rows)
        j._refs = bufs
        j.in_elems = m.in_elems
        return j

    def close(self) -> None:
        if self.handle:
            self.lib.qm_store_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceBuffer:
    """A device allocation made by the library (freed with qm_device_free)."""

    def __init__(self, rt: "Runtime", ptr: int, nbytes: int):
        self.rt = rt
        self.ptr = ptr
        self.nbytes = nbytes
        rt._children.add(self)

    def data_ptr(self) -> int:
        return self.ptr

    def close(self) -> None:
        if self.ptr:
            self.rt.lib.qm_device_free(self.rt.handle, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
