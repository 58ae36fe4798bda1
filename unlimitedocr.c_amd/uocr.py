"""ctypes host binding of libunlimitedocr.so (MI355X build).

Mirrors the reference's Python bridge (src/unlimitedocr_c/ffi.py): the same
struct layouts (ffi.py CEngineOpts / CPreparedRequest / CImageView /
CMemoryReport / CProfileReport), the same exported functions
(ffi.py:305-335), an ``Engine`` whose ``generate_prepared`` returns the
generated ids and raises ``RuntimeError`` with the engine's error text on a
non-OK status (ffi.py:681-699), and a per-engine lock (ffi.py:691).

MI355X additions: ``Engine.from_memory`` / ``Engine.generate_embeddings``
(precomputed image rows, include/uocr_hip.h), the hot-path operators on
device buffers (``DeviceBuffer`` and the ``op_*`` functions) and the
synthetic model builder (``synth_model``).  The library must be built
(``make -C unlimitedocr.c_amd``); there is no fallback implementation.
"""
from __future__ import annotations

import ctypes as ct
import os
import threading
from pathlib import Path

import numpy as np

PACKAGE_DIR = Path(__file__).resolve().parent
LIBRARY_PATH = PACKAGE_DIR / "lib" / "libunlimitedocr.so"

UOCR_OK = 0
UOCR_ERROR_INVALID_ARGUMENT = -1
UOCR_ERROR_UNSUPPORTED = -2
UOCR_ERROR_OUT_OF_MEMORY = -3
UOCR_ERROR_NOT_IMPLEMENTED = -4
UOCR_ERROR_INTERNAL = -5
UOCR_MEMORY_CATEGORY_COUNT = 10
UOCR_PROFILE_MAX_EVENTS = 256

QT_F16, QT_Q8, QT_Q4 = 1, 3, 4
QPROFILE_FP16, QPROFILE_Q8, QPROFILE_Q4 = 1, 2, 3
GEN_IGNORE_EOS, GEN_NO_GRAPH, GEN_TOKEN_PREFILL, GEN_NO_RUN = 1, 2, 4, 8

HIDDEN, VOCAB, HEADS, HEAD_DIM = 1280, 129280, 10, 128
TOKEN_BOS, TOKEN_EOS, TOKEN_IMAGE = 0, 1, 128815


class CImageView(ct.Structure):
    _fields_ = [("pixels", ct.c_void_p), ("width", ct.c_uint32), ("height", ct.c_uint32),
                ("format", ct.c_int), ("kind", ct.c_int)]


class CPreparedRequest(ct.Structure):
    _fields_ = [("input_ids", ct.POINTER(ct.c_int32)), ("image_mask", ct.POINTER(ct.c_uint8)),
                ("n_tokens", ct.c_uint32), ("views", ct.POINTER(CImageView)), ("n_views", ct.c_uint32),
                ("crop_grid_w", ct.c_uint32), ("crop_grid_h", ct.c_uint32), ("max_new_tokens", ct.c_uint32)]


class CEngineOpts(ct.Structure):
    _fields_ = [("model_path", ct.c_char_p), ("backend", ct.c_char_p), ("resource_path", ct.c_char_p),
                ("max_batch", ct.c_uint32), ("max_prompt_tokens", ct.c_uint32), ("max_gen_tokens", ct.c_uint32),
                ("profile", ct.c_uint32), ("reserved0", ct.c_uint32), ("memory_budget_bytes", ct.c_uint64)]


class CProfileEvent(ct.Structure):
    _fields_ = [("name", ct.c_char * 64), ("calls", ct.c_uint64), ("total_ms", ct.c_double),
                ("min_ms", ct.c_double), ("max_ms", ct.c_double)]


class CMemoryReport(ct.Structure):
    _fields_ = [("category_live_bytes", ct.c_uint64 * UOCR_MEMORY_CATEGORY_COUNT),
                ("category_peak_bytes", ct.c_uint64 * UOCR_MEMORY_CATEGORY_COUNT)] + [
        (name, ct.c_uint64) for name in (
            "total_live_bytes", "total_peak_bytes", "estimated_model_views_bytes", "estimated_kv_cache_bytes",
            "estimated_prompt_embeddings_bytes", "estimated_vision_scratch_bytes",
            "estimated_vision_gpu_workspace_bytes", "estimated_vision_final_features_bytes",
            "estimated_vision_host_staging_bytes", "estimated_decoder_scratch_bytes", "estimated_moe_scratch_bytes",
            "estimated_logits_readback_bytes", "estimated_transient_bytes", "estimated_safety_margin_bytes",
            "estimated_total_bytes", "memory_budget_bytes", "recommended_working_set_bytes",
            "vision_workspace_capacity_bytes", "vision_workspace_high_watermark_bytes")]


class CProfileReport(ct.Structure):
    _fields_ = [("enabled", ct.c_uint32), ("event_count", ct.c_uint32), ("dropped_event_count", ct.c_uint32),
                ("reserved0", ct.c_uint32), ("generation_index", ct.c_uint64),
                ("events", CProfileEvent * UOCR_PROFILE_MAX_EVENTS)] + [
        (name, ct.c_uint64) for name in (
            "metal_buffer_allocation_count", "metal_buffer_allocation_bytes", "metal_command_buffer_count",
            "metal_command_encoder_count", "metal_command_buffer_wait_count", "metal_mps_descriptor_count",
            "metal_mps_ndarray_count", "metal_nsarray_count", "metal_transient_retain_object_count")] + [
        ("memory", CMemoryReport)]


class CMoeWeights(ct.Structure):
    _fields_ = [("router", ct.c_void_p), ("expert_qtype", ct.c_uint32),
                ("gate_w", ct.c_void_p), ("gate_s", ct.c_void_p), ("up_w", ct.c_void_p), ("up_s", ct.c_void_p),
                ("gu_w_stride", ct.c_uint64), ("gu_s_stride", ct.c_uint64),
                ("down_w", ct.c_void_p), ("down_s", ct.c_void_p),
                ("dn_w_stride", ct.c_uint64), ("dn_s_stride", ct.c_uint64),
                ("shared_qtype", ct.c_uint32),
                ("sgate_w", ct.c_void_p), ("sgate_s", ct.c_void_p), ("sup_w", ct.c_void_p), ("sup_s", ct.c_void_p),
                ("sdown_w", ct.c_void_p), ("sdown_s", ct.c_void_p)]


# Exported symbols of include/unlimitedocr.h, include/uocr_hip.h and
# include/uocr_synth.h: name -> (argtypes, restype).
_VP, _U32, _I32, _SZ = ct.c_void_p, ct.c_uint32, ct.c_int32, ct.c_size_t
SIGNATURES = {
    "uocr_abi_version": ([], ct.c_uint32),
    "uocr_status_string": ([ct.c_int], ct.c_char_p),
    "uocr_engine_open": ([ct.POINTER(CEngineOpts)], _VP),
    "uocr_engine_close": ([_VP], None),
    "uocr_last_error": ([_VP], ct.c_char_p),
    "uocr_engine_backend": ([_VP], ct.c_char_p),
    "uocr_memory_category_name": ([ct.c_int], ct.c_char_p),
    "uocr_engine_memory_report": ([_VP, ct.POINTER(CMemoryReport)], ct.c_int),
    "uocr_engine_profile_report": ([_VP, ct.POINTER(CProfileReport)], ct.c_int),
    "uocr_engine_profile_reset": ([_VP], ct.c_int),
    "uocr_generate_prepared": ([_VP, ct.POINTER(CPreparedRequest), _U32, ct.POINTER(_VP)], ct.c_int),
    "uocr_result_count": ([_VP], ct.c_uint32),
    "uocr_result_tokens": ([_VP, _U32, ct.POINTER(_U32)], ct.POINTER(ct.c_int32)),
    "uocr_result_free": ([_VP], None),
    "uocr_engine_open_memory": ([ct.POINTER(CEngineOpts), _VP, _SZ], _VP),
    "uocr_generate_embeddings": ([_VP, _VP, _VP, _VP, _U32, _U32, _U32, _U32, _VP, _VP, ct.POINTER(_U32),
                                  ct.POINTER(ct.c_double), ct.POINTER(ct.c_double)], ct.c_int),
    "uocr_engine_trace_enable": ([_VP, _U32], ct.c_int),
    "uocr_engine_trace_read": ([_VP, _VP, _VP], ct.c_int),
    "uocr_engine_trace_force": ([_VP, _VP, _U32], ct.c_int),
    "uocr_engine_trace_read_weights": ([_VP, _VP], ct.c_int),
    "uocr_engine_trace_read_router_inputs": ([_VP, _VP], ct.c_int),
    "uocr_engine_decode_path": ([_VP], ct.c_int),
    "uocr_op_workspace_bytes": ([], _SZ),
    "uocr_op_gemv": ([_U32, _VP, _VP, _U32, _U32, _VP, _VP, _VP], ct.c_int),
    "uocr_op_swiglu": ([_U32, _VP, _VP, _VP, _VP, _U32, _U32, _VP, _VP, _VP], ct.c_int),
    "uocr_op_rmsnorm": ([_VP, _VP, _U32, _VP], ct.c_int),
    "uocr_op_lm_head_argmax": ([_U32, _VP, _VP, _U32, _VP, _VP, _VP, _VP, _VP], ct.c_int),
    "uocr_op_lm_head_keys": ([_U32, _VP, _VP, _U32, _VP, _VP, _VP], ct.c_int),
    "uocr_op_router": ([_VP, _VP, _VP, ct.c_int, _VP, _VP, _VP], ct.c_int),
    "uocr_op_moe_ffn": ([ct.POINTER(CMoeWeights), _VP, _VP, _VP, ct.c_int, _VP, _VP, _VP, _VP], ct.c_int),
    "uocr_op_moe_gate_up": ([ct.POINTER(CMoeWeights), _VP, _VP, _VP, ct.c_int, _VP, _VP, _VP, _VP], ct.c_int),
    "uocr_op_attention_decode": ([_VP, _VP, _VP, _U32, _U32, _U32, _VP, _VP], ct.c_int),
    "uocr_op_attention_block": ([_U32, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _U32, _U32,
                                 _U32, _VP, _VP], ct.c_int),
    "uocr_op_embed": ([_U32, _VP, _VP, _U32, _VP, _VP], ct.c_int),
    "uocr_op_gemm": ([_U32, _VP, _VP, _U32, _U32, _U32, _VP, _VP, _VP], ct.c_int),
    "uocr_op_vision_linear": ([_U32, _VP, _VP, _VP, _U32, _U32, _U32, _U32, _U32, _VP, _VP, _VP, _VP], ct.c_int),
    "uocr_op_prefill_attention": ([_VP, _VP, _VP, _U32, _U32, _VP], ct.c_int),
    "uocr_op_moe_rows_workspace_bytes": ([_U32], _SZ),
    "uocr_op_moe_ffn_rows": ([ct.POINTER(CMoeWeights), _VP, _VP, _VP, _U32, ct.c_int, _VP, _VP], ct.c_int),
    "uocr_op_moe_ffn_rows_static": ([ct.POINTER(CMoeWeights), _VP, _VP, _VP, _U32, ct.c_int, _VP], ct.c_int),
    "uocr_hip_device_count": ([], ct.c_int),
    "uocr_hip_alloc": ([_SZ], _VP),
    "uocr_hip_free": ([_VP], ct.c_int),
    "uocr_hip_upload": ([_VP, _VP, _SZ], ct.c_int),
    "uocr_hip_download": ([_VP, _VP, _SZ], ct.c_int),
    "uocr_hip_memset": ([_VP, ct.c_int, _SZ], ct.c_int),
    "uocr_hip_copy": ([_VP, _VP, _SZ], ct.c_int),
    "uocr_hip_sync": ([], ct.c_int),
    "uocr_hip_op_error": ([], ct.c_char_p),
    "uocr_hip_timer_begin": ([], ct.c_int),
    "uocr_hip_timer_end_ms": ([], ct.c_float),
    "uocr_hip_capture_begin": ([], ct.c_int),
    "uocr_hip_capture_end": ([], ct.c_int),
    "uocr_hip_graph_replay": ([ct.c_uint32], ct.c_int),
    "uocr_hip_graph_release": ([], ct.c_int),
    "uocr_synth_model_build": ([_U32, ct.c_uint64, ct.POINTER(_VP), ct.POINTER(_SZ)], ct.c_int),
    "uocr_synth_model_write": ([ct.c_char_p, _U32, ct.c_uint64], ct.c_int),
    "uocr_synth_free": ([_VP], None),
    "uocr_quantize_rows": ([_U32, _VP, _U32, _U32, _VP, _VP], ct.c_int),
    "uocr_image_skeleton_build": ([_U32, ct.POINTER(_VP), ct.POINTER(_SZ)], ct.c_int),
}

_LIB: ct.CDLL | None = None
_LIB_LOCK = threading.Lock()


def library_path() -> Path:
    env = os.environ.get("UOCR_LIBRARY_PATH")
    return Path(env) if env else LIBRARY_PATH


def load_library() -> ct.CDLL:
    """Load and bind libunlimitedocr.so; raises if it has not been built."""
    global _LIB
    with _LIB_LOCK:
        if _LIB is None:
            path = library_path()
            if not path.exists():
                raise FileNotFoundError(f"{path} is not built; run `make -C unlimitedocr.c_amd`")
            lib = ct.CDLL(str(path))
            for name, (args, res) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = res
            _LIB = lib
        return _LIB


def _check_op(status: int, what: str) -> None:
    if status != UOCR_OK:
        msg = load_library().uocr_hip_op_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({status}): {msg}")


# ---------------------------------------------------------------------------
# engine (ffi.py Engine)
# ---------------------------------------------------------------------------

class Engine:
    """One uocr_engine; calls are serialised by a per-engine lock."""

    def __init__(self, model_path: str | None = None, backend: str = "auto", *, max_prompt_tokens: int = 0,
                 max_gen_tokens: int = 0, max_batch: int = 0, profile: bool = False, memory_budget_bytes: int = 0,
                 _memory: tuple[int, int] | None = None) -> None:
        self._lib = load_library()
        self._lock = threading.Lock()
        self._keep = None
        opts = CEngineOpts(model_path.encode() if model_path else None, backend.encode() if backend else None, None,
                           max_batch, max_prompt_tokens, max_gen_tokens, 1 if profile else 0, 0, memory_budget_bytes)
        if _memory is not None:
            handle = self._lib.uocr_engine_open_memory(ct.byref(opts), ct.c_void_p(_memory[0]), _memory[1])
        else:
            handle = self._lib.uocr_engine_open(ct.byref(opts))
        if not handle:
            raise RuntimeError(self._lib.uocr_last_error(None).decode(errors="replace"))
        self._handle = ct.c_void_p(handle)

    @classmethod
    def from_memory(cls, image: "SynthModel", backend: str = "hip", **kw) -> "Engine":
        eng = cls(None, backend, _memory=(image.ptr, image.size), **kw)
        eng._keep = image
        return eng

    def close(self) -> None:
        with self._lock:
            if self._handle:
                self._lib.uocr_engine_close(self._handle)
                self._handle = ct.c_void_p(None)

    def __enter__(self) -> "Engine":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    @property
    def backend(self) -> str:
        return self._lib.uocr_engine_backend(self._handle).decode()

    def last_error(self) -> str:
        return self._lib.uocr_last_error(self._handle).decode(errors="replace")

    def memory_report(self) -> CMemoryReport:
        rep = CMemoryReport()
        self._raise(self._lib.uocr_engine_memory_report(self._handle, ct.byref(rep)))
        return rep

    def profile_report(self) -> CProfileReport:
        rep = CProfileReport()
        self._raise(self._lib.uocr_engine_profile_report(self._handle, ct.byref(rep)))
        return rep

    def profile_reset(self) -> None:
        self._raise(self._lib.uocr_engine_profile_reset(self._handle))

    def profile_events(self) -> dict[str, tuple[int, float]]:
        rep = self.profile_report()
        return {rep.events[i].name.decode(): (rep.events[i].calls, rep.events[i].total_ms)
                for i in range(rep.event_count)}

    def _raise(self, status: int) -> None:
        if status != UOCR_OK:
            err = RuntimeError(f"{self._lib.uocr_status_string(status).decode()}: {self.last_error()}")
            err.status = status  # type: ignore[attr-defined]
            raise err

    def generate_prepared(self, input_ids, image_mask=None, max_new_tokens: int = 1, views=None) -> np.ndarray:
        ids = np.ascontiguousarray(input_ids, dtype=np.int32)
        mask = np.zeros(ids.shape, np.uint8) if image_mask is None else np.ascontiguousarray(image_mask, np.uint8)
        req = CPreparedRequest(ids.ctypes.data_as(ct.POINTER(ct.c_int32)), mask.ctypes.data_as(ct.POINTER(ct.c_uint8)),
                               ids.size, None, 0, 1, 1, max_new_tokens)
        out = ct.c_void_p()
        with self._lock:
            self._raise(self._lib.uocr_generate_prepared(self._handle, ct.byref(req), 1, ct.byref(out)))
        try:
            n = ct.c_uint32()
            ptr = self._lib.uocr_result_tokens(out, 0, ct.byref(n))
            return np.ctypeslib.as_array(ptr, shape=(n.value,)).copy() if n.value else np.zeros(0, np.int32)
        finally:
            self._lib.uocr_result_free(out)

    def generate_embeddings(self, input_ids, image_mask=None, image_rows=None, max_new_tokens: int = 1,
                            flags: int = 0) -> tuple[np.ndarray, np.ndarray, float, float]:
        """Returns (ids, scores, prefill_ms, decode_ms)."""
        ids = np.ascontiguousarray(input_ids, dtype=np.int32)
        mask = None if image_mask is None else np.ascontiguousarray(image_mask, np.uint8)
        rows = None if image_rows is None else np.ascontiguousarray(image_rows, np.float16)
        n_rows = 0 if rows is None else rows.shape[0]
        out = np.zeros(max_new_tokens, np.int32)
        scores = np.zeros(max_new_tokens, np.float32)
        count = ct.c_uint32()
        pre, dec = ct.c_double(), ct.c_double()
        with self._lock:
            self._raise(self._lib.uocr_generate_embeddings(
                self._handle, ids.ctypes.data, None if mask is None else mask.ctypes.data,
                None if rows is None else rows.ctypes.data, n_rows, ids.size, max_new_tokens, flags,
                out.ctypes.data, scores.ctypes.data, ct.byref(count), ct.byref(pre), ct.byref(dec)))
        return out[:count.value], scores[:count.value], pre.value, dec.value

    def trace_enable(self, steps: int) -> None:
        """Record the router selections of the first `steps` decode steps of
        each following generation (0 turns tracing off)."""
        with self._lock:
            self._raise(self._lib.uocr_engine_trace_enable(self._handle, steps))
        self._trace_steps = steps

    def trace_force(self, ids) -> None:
        """Embed ids[t] after decode step t of each following generation
        (teacher forcing); an empty sequence turns it off."""
        arr = np.ascontiguousarray(ids if ids is not None else [], dtype=np.int32)
        with self._lock:
            self._raise(self._lib.uocr_engine_trace_force(self._handle, arr.ctypes.data if arr.size else None,
                                                          arr.size))

    def trace_read(self) -> tuple[np.ndarray, np.ndarray]:
        """(expert ids [steps][11][6] uint32, final hidden state fp16 [1280])
        of the last generation."""
        steps = getattr(self, "_trace_steps", 0)
        ids = np.zeros((steps, 11, 6), np.uint32)
        hidden = np.zeros(1280, np.float16)
        with self._lock:
            self._raise(self._lib.uocr_engine_trace_read(self._handle, ids.ctypes.data if steps else None,
                                                         hidden.ctypes.data))
        return ids, hidden

    def trace_read_weights(self) -> np.ndarray:
        """Routing weights [steps][11][6] float32 of the traced selections
        (selection order, NaN for steps the last generation did not reach)."""
        steps = getattr(self, "_trace_steps", 0)
        w = np.zeros((steps, 11, 6), np.float32)
        if steps:
            with self._lock:
                self._raise(self._lib.uocr_engine_trace_read_weights(self._handle, w.ctypes.data))
        return w

    def trace_read_router_inputs(self) -> np.ndarray:
        """Router inputs [steps][11][1280] (fp16 bits as uint16) of the traced
        selections: the pre-norm input a = h + O ctx of each MoE layer."""
        steps = getattr(self, "_trace_steps", 0)
        a = np.zeros((steps, 11, 1280), np.uint16)
        if steps:
            with self._lock:
                self._raise(self._lib.uocr_engine_trace_read_router_inputs(self._handle, a.ctypes.data))
        return a

    def decode_path(self) -> int:
        """1: the last generation decoded on the persistent run; 0: on the
        per-step kernels; 2: per-step kernels after the run gave up waiting;
        -1: no generation yet."""
        with self._lock:
            return int(self._lib.uocr_engine_decode_path(self._handle))


# ---------------------------------------------------------------------------
# synthetic .uocr images
# ---------------------------------------------------------------------------

class SynthModel:
    """A synthetic .uocr image in library-owned host memory."""

    def __init__(self, qprofile: int, seed: int | None) -> None:
        """seed None: the zero-filled skeleton the converter fills
        (uocr_image_skeleton_build), else the seeded synthetic values."""
        self._lib = load_library()
        ptr, size = ct.c_void_p(), ct.c_size_t()
        if seed is None:
            status = self._lib.uocr_image_skeleton_build(qprofile, ct.byref(ptr), ct.byref(size))
        else:
            status = self._lib.uocr_synth_model_build(qprofile, seed, ct.byref(ptr), ct.byref(size))
        if status != UOCR_OK:
            raise RuntimeError(f"model image build failed ({status})")
        self.ptr, self.size, self.qprofile, self.seed = ptr.value, size.value, qprofile, seed

    def view(self) -> np.ndarray:
        return np.ctypeslib.as_array((ct.c_uint8 * self.size).from_address(self.ptr))

    def close(self) -> None:
        if self.ptr:
            self._lib.uocr_synth_free(ct.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


TENSOR_ENTRY = np.dtype([("id", "<u4"), ("family", "<u4"), ("layer", "<i4"), ("expert", "<i4"),
                         ("projection", "<u4"), ("usage", "<u4"), ("qtype", "<u4"), ("flags", "<u4"), ("rank", "<u4"),
                         ("lshape", "<u4", 4), ("pshape", "<u4", 4), ("payload_offset", "<u8"),
                         ("payload_size", "<u8"), ("block_size", "<u4"), ("row_size", "<u4"),
                         ("scale_offset", "<u8"), ("scale_size", "<u8"), ("min_offset", "<u8"), ("min_size", "<u8"),
                         ("reasons", "<u4", 2), ("source_name", "<u4", 2)])
assert TENSOR_ENTRY.itemsize == 140


def tensor_table(image: np.ndarray) -> np.ndarray:
    """Tensor directory of a .uocr image in memory (uint8 array), the entry
    layout of include/uocr_format.h (uocr_format.h:268-299 in the reference)."""
    hdr = image[:112]
    n_sec = int(hdr[24:28].view("<u4")[0])
    sec_off = int(hdr[40:48].view("<u8")[0])
    secs = image[sec_off:sec_off + 32 * n_sec].view(np.dtype([("type", "<u4"), ("flags", "<u4"), ("offset", "<u8"),
                                                                ("size", "<u8"), ("alignment", "<u8")]))
    d = secs[secs["type"] == 2][0]
    count = int(image[d["offset"] + 12:d["offset"] + 16].view("<u4")[0])
    start = int(d["offset"]) + 16
    return image[start:start + 140 * count].view(TENSOR_ENTRY)


def f16_tensor(image: np.ndarray, entry, rows: int, cols: int) -> np.ndarray:
    """fp16 payload of a tensor entry as a [rows][cols] float16 view."""
    off, size = int(entry["payload_offset"]), int(entry["payload_size"])
    assert size == rows * cols * 2, (int(entry["id"]), size, rows, cols)
    return image[off:off + size].view(np.float16).reshape(rows, cols)


def synth_model(qprofile: int, seed: int) -> SynthModel:
    return SynthModel(qprofile, seed)


# ---------------------------------------------------------------------------
# device buffers and operators
# ---------------------------------------------------------------------------

class DeviceBuffer:
    """hipMalloc'd device memory owned by Python."""

    def __init__(self, nbytes: int) -> None:
        self._lib = load_library()
        self.nbytes = int(nbytes)
        self.ptr = self._lib.uocr_hip_alloc(max(self.nbytes, 1))
        if not self.ptr:
            raise MemoryError(self._lib.uocr_hip_op_error().decode())

    @classmethod
    def of(cls, array: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(array)
        buf = cls(arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, array: np.ndarray) -> None:
        arr = np.ascontiguousarray(array)
        assert arr.nbytes <= self.nbytes
        _check_op(self._lib.uocr_hip_upload(ct.c_void_p(self.ptr), arr.ctypes.data, arr.nbytes), "upload")

    def download(self, dtype, count: int | None = None) -> np.ndarray:
        dt = np.dtype(dtype)
        n = self.nbytes // dt.itemsize if count is None else count
        out = np.empty(n, dt)
        _check_op(self._lib.uocr_hip_download(out.ctypes.data, ct.c_void_p(self.ptr), out.nbytes), "download")
        return out

    def zero(self) -> None:
        _check_op(self._lib.uocr_hip_memset(ct.c_void_p(self.ptr), 0, self.nbytes), "memset")

    def free(self) -> None:
        if self.ptr:
            self._lib.uocr_hip_free(ct.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self) -> None:
        try:
            self.free()
        except Exception:
            pass


def _p(buf) -> ct.c_void_p:
    if buf is None:
        return ct.c_void_p(None)
    if isinstance(buf, DeviceBuffer):
        return ct.c_void_p(buf.ptr)
    return ct.c_void_p(int(buf))


def copy(dst, src, nbytes: int) -> None:
    """Device-to-device copy on the operator stream."""
    _check_op(load_library().uocr_hip_copy(_p(dst), _p(src), nbytes), "copy")


def sync() -> None:
    _check_op(load_library().uocr_hip_sync(), "sync")


def workspace() -> DeviceBuffer:
    return DeviceBuffer(load_library().uocr_op_workspace_bytes())


def op_gemv(qtype, w, s, rows, k, x, residual, y) -> None:
    _check_op(load_library().uocr_op_gemv(qtype, _p(w), _p(s), rows, k, _p(x), _p(residual), _p(y)), "op_gemv")


def op_swiglu(qtype, gw, gs, uw, us, rows, k, x, norm_w, mid) -> None:
    _check_op(load_library().uocr_op_swiglu(qtype, _p(gw), _p(gs), _p(uw), _p(us), rows, k, _p(x), _p(norm_w),
                                            _p(mid)), "op_swiglu")


def op_rmsnorm(x, w, n, y) -> None:
    _check_op(load_library().uocr_op_rmsnorm(_p(x), _p(w), n, _p(y)), "op_rmsnorm")


def op_lm_head_argmax(qtype, w, s, vocab, x, norm_w, ws, token, score) -> None:
    _check_op(load_library().uocr_op_lm_head_argmax(qtype, _p(w), _p(s), vocab, _p(x), _p(norm_w), _p(ws), _p(token),
                                                    _p(score)), "op_lm_head_argmax")


def op_lm_head_keys(qtype, w, s, vocab, x, norm_w, keys) -> None:
    _check_op(load_library().uocr_op_lm_head_keys(qtype, _p(w), _p(s), vocab, _p(x), _p(norm_w), _p(keys)),
              "op_lm_head_keys")


def op_router(router, x, norm_w, norm_topk, ws, ids, weights) -> None:
    _check_op(load_library().uocr_op_router(_p(router), _p(x), _p(norm_w), norm_topk, _p(ws), _p(ids), _p(weights)),
              "op_router")


def op_moe_ffn(weights: CMoeWeights, x, norm_w, residual, norm_topk, ws, out, ids, wts) -> None:
    _check_op(load_library().uocr_op_moe_ffn(ct.byref(weights), _p(x), _p(norm_w), _p(residual), norm_topk, _p(ws),
                                             _p(out), _p(ids), _p(wts)), "op_moe_ffn")


def op_moe_gate_up(weights: CMoeWeights, logits, x, norm_w, norm_topk, mid, smid, ids, wts) -> None:
    _check_op(load_library().uocr_op_moe_gate_up(ct.byref(weights), _p(logits), _p(x), _p(norm_w), norm_topk,
                                                 _p(mid), _p(smid), _p(ids), _p(wts)), "op_moe_gate_up")


def op_attention_decode(q, kc, vc, cap, prompt_len, gen, ws, out) -> None:
    _check_op(load_library().uocr_op_attention_decode(_p(q), _p(kc), _p(vc), cap, prompt_len, gen, _p(ws), _p(out)),
              "op_attention_decode")


def op_attention_block(qtype, wq, sq, wk, sk, wv, sv, wo, so, hidden, norm_w, kc, vc, cap, prompt_len, gen, ws,
                       out) -> None:
    _check_op(load_library().uocr_op_attention_block(qtype, _p(wq), _p(sq), _p(wk), _p(sk), _p(wv), _p(sv), _p(wo),
                                                     _p(so), _p(hidden), _p(norm_w), _p(kc), _p(vc), cap, prompt_len,
                                                     gen, _p(ws), _p(out)), "op_attention_block")


def op_embed(qtype, w, s, vocab, token, out) -> None:
    _check_op(load_library().uocr_op_embed(qtype, _p(w), _p(s), vocab, _p(token), _p(out)), "op_embed")


def op_gemm(qtype, w, s, m, n, k, x, residual, y) -> None:
    _check_op(load_library().uocr_op_gemm(qtype, _p(w), _p(s), m, n, k, _p(x), _p(residual), _p(y)), "op_gemm")


VISION_ACT_NONE, VISION_ACT_QUICKGELU, VISION_ACT_GELU_ERF = 0, 1, 2


def op_vision_linear(qtype, w, s, bias, m, k, n, act, split, x, dst0, dst1=None, dst2=None) -> None:
    """dst = f16(act(x . W^T + bias)); split != 0 routes column thirds to dst0/dst1/dst2."""
    _check_op(load_library().uocr_op_vision_linear(qtype, _p(w), _p(s), _p(bias), m, k, n, act, split, _p(x),
                                                   _p(dst0), _p(dst1), _p(dst2)), "op_vision_linear")


def op_prefill_attention(q, kc, vc, cap, prompt_len, ctx) -> None:
    _check_op(load_library().uocr_op_prefill_attention(_p(q), _p(kc), _p(vc), cap, prompt_len, _p(ctx)),
              "op_prefill_attention")


def moe_rows_workspace(rows: int) -> DeviceBuffer:
    return DeviceBuffer(load_library().uocr_op_moe_rows_workspace_bytes(rows))


def op_moe_ffn_rows(weights: CMoeWeights, x, norm_w, residual, rows, norm_topk, ws, out) -> None:
    _check_op(load_library().uocr_op_moe_ffn_rows(ct.byref(weights), _p(x), _p(norm_w), _p(residual), rows, norm_topk,
                                                  _p(ws), _p(out)), "op_moe_ffn_rows")


STATIC_MAX_ROWS = 64


def op_moe_ffn_rows_static(weights: CMoeWeights, x, norm_w, residual, rows, norm_topk, out) -> None:
    """uocr_op_moe_ffn_rows on the library's static scratch (no workspace, no
    device allocation; rows <= STATIC_MAX_ROWS)."""
    _check_op(load_library().uocr_op_moe_ffn_rows_static(ct.byref(weights), _p(x), _p(norm_w), _p(residual), rows,
                                                         norm_topk, _p(out)), "op_moe_ffn_rows_static")


class Timer:
    """hipEvent timer on the operator stream."""

    def __enter__(self) -> "Timer":
        _check_op(load_library().uocr_hip_timer_begin(), "timer begin")
        return self

    def __exit__(self, *exc) -> None:
        self.ms = float(load_library().uocr_hip_timer_end_ms())


class Capture:
    """Records the operator calls made inside the block into one hipGraph
    (uocr_hip_capture_begin/end); `replay(n)` launches it n times."""

    def __enter__(self) -> "Capture":
        _check_op(load_library().uocr_hip_capture_begin(), "capture begin")
        return self

    def __exit__(self, exc_type, *exc) -> None:
        status = load_library().uocr_hip_capture_end()
        if exc_type is None:
            _check_op(status, "capture end")

    def replay(self, times: int = 1) -> None:
        _check_op(load_library().uocr_hip_graph_replay(times), "graph replay")

    def release(self) -> None:
        load_library().uocr_hip_graph_release()
