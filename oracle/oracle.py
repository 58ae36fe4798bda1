"""ctypes binding of the CPU oracle (liboracle.so) and of the reference's own
CPU path compiled from its sources (_ref/libuocr_cpu_ref.so, when built).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg.  The product never imports this module.
"""
from __future__ import annotations

import ctypes as ct
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
ORACLE_LIB = ORACLE_DIR / "liboracle.so"
REF_LIB = ORACLE_DIR / "_ref" / "libuocr_cpu_ref.so"

_VP, _U32, _I32, _F = ct.c_void_p, ct.c_uint32, ct.c_int32, ct.c_float


class Plan(ct.Structure):
    _fields_ = [(n, ct.c_uint32) for n in ("prompt_length", "generated_count", "live_generated",
                                           "first_generated_index", "query_position", "attention_length",
                                           "ring_window")]


class ExpertView(ct.Structure):
    _fields_ = [("qtype", ct.c_uint32), ("gate_w", _VP), ("gate_s", _VP), ("up_w", _VP), ("up_s", _VP),
                ("down_w", _VP), ("down_s", _VP), ("w_stride", ct.c_uint64), ("s_stride", ct.c_uint64)]


_SIGS = {
    "orc_f16_to_f32": ([ct.c_uint16], _F),
    "orc_f32_to_f16": ([_F], ct.c_uint16),
    "orc_bf16_to_f32": ([ct.c_uint16], _F),
    "orc_rmsnorm_f32": ([_VP, _VP, _U32, _U32, _F, _VP], ct.c_int),
    "orc_rope_split_half_f32": ([_VP, _VP, _U32, _U32, _U32, _U32, _F, _VP, _VP], ct.c_int),
    "orc_causal_sdpa_f32": ([_VP, _VP, _VP, _U32, _U32, _U32, _F, _VP], ct.c_int),
    "orc_dense_swiglu_f32": ([_VP, _VP, _VP, _VP, _U32, _U32, _U32, _VP, _VP], ct.c_int),
    "orc_moe_router_f32": ([_VP, _VP, _U32, _U32, _U32, _U32, _F, _VP, _VP, _VP, _VP], ct.c_int),
    "orc_moe_swiglu_f32": ([_VP] * 8 + [_U32] * 6 + [_F] + [_VP] * 7, ct.c_int),
    "orc_kv_cache_token_for_position": ([_U32, _U32, _U32, _U32, ct.POINTER(_U32)], ct.c_int),
    "orc_decode_attention_plan": ([_U32, _U32, _U32, _U32, ct.POINTER(Plan)], ct.c_int),
    "orc_attention_index_to_token": ([ct.POINTER(Plan), _U32, ct.POINTER(_U32)], ct.c_int),
    "orc_row_dot": ([_U32, _VP, _VP, _U32, _U32, _VP], _F),
    "orc_weight_at": ([_U32, _VP, _VP, _U32, _U32, _U32], _F),
    "orc_gemv": ([_U32, _VP, _VP, _U32, _U32, _VP, _VP, _VP], ct.c_int),
    "orc_swiglu_mid": ([_U32, _VP, _VP, _VP, _VP, _U32, _U32, _VP, _VP], ct.c_int),
    "orc_rmsnorm_f16": ([_VP, _VP, _U32, _F, _VP], ct.c_int),
    "orc_rope_f16": ([_VP, _VP, _U32, _U32, _U32, _F], ct.c_int),
    "orc_lm_head_argmax": ([_U32, _VP, _VP, _U32, _U32, _VP, ct.POINTER(_I32), ct.POINTER(_F), ct.POINTER(_F)],
                           ct.c_int),
    "orc_router_topk": ([_VP, _VP, _U32, _U32, _U32, ct.c_int, _VP, _VP, _VP, _VP], ct.c_int),
    "orc_moe_ffn": ([_VP, _VP, _VP, _U32, _U32, ct.c_int, ct.POINTER(ExpertView), _U32, _U32, _VP, _VP, _VP, _VP,
                     _VP, _VP, _U32, _VP, _VP, _VP, _VP], ct.c_int),
    "orc_attention_decode": ([_VP, _VP, _VP, _U32, _U32, ct.POINTER(Plan), _VP], ct.c_int),
    "orc_embed_row": ([_U32, _VP, _VP, _U32, _U32, _I32, _VP], ct.c_int),
    "orc_session_embed": ([_VP, _I32, _VP], ct.c_int),
    "orc_model_open": ([_VP, ct.c_size_t, ct.c_char_p, ct.c_size_t], _VP),
    "orc_model_close": ([_VP], None),
    "orc_session_create": ([_VP, _U32], _VP),
    "orc_session_destroy": ([_VP], None),
    "orc_generate": ([_VP, _VP, _VP, _VP, _U32, _U32, ct.c_int, _VP, _VP], ct.c_int),
    "orc_session_reset": ([_VP, _U32], ct.c_int),
    "orc_forward_token": ([_VP, _VP, _U32, _VP], ct.c_int),
    "orc_forward_token_traced": ([_VP, _VP, _U32, _VP, _VP, _VP], ct.c_int),
    "orc_select": ([_VP, _VP, ct.POINTER(_I32), ct.POINTER(_F), ct.POINTER(_F)], ct.c_int),
    "orc_session_fill_kv": ([_VP, _U32, ct.c_uint64], ct.c_int),
    "orc_vision_linear": ([_U32, _VP, _VP, _VP, _U32, _U32, _U32, _U32, _U32, _VP, _VP, _VP, _VP], ct.c_int),
    "orc_set_threads": ([ct.c_int], None),
    "orc_get_threads": ([], ct.c_int),
}

_LIB: ct.CDLL | None = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)


def lib() -> ct.CDLL:
    global _LIB
    if _LIB is None:
        if not ORACLE_LIB.exists():
            build()
        l = ct.CDLL(str(ORACLE_LIB))
        for name, (args, res) in _SIGS.items():
            f = getattr(l, name)
            f.argtypes = args
            f.restype = res
        _LIB = l
    return _LIB


def ref_lib() -> ct.CDLL | None:
    """The reference's uocr_cpu_ref.c built from its own source (or None)."""
    return ct.CDLL(str(REF_LIB)) if REF_LIB.exists() else None


def ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def f16_bits(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, np.float16)).view(np.uint16)


def gemv(qtype, W, S, rows, K, x_bits, residual_bits=None) -> np.ndarray:
    y = np.zeros(rows, np.uint16)
    assert lib().orc_gemv(qtype, ptr(W), ptr(S), rows, K, ptr(x_bits), ptr(residual_bits), ptr(y)) == 1
    return y


def vision_linear(qtype, W, S, bias_bits, m, K, N, act, split, x_bits):
    """f16 bits [m][N] (split == 0) or a tuple of three [m][split] arrays."""
    x_bits = np.ascontiguousarray(x_bits, np.uint16)
    if split == 0:
        out = np.zeros((m, N), np.uint16)
        assert lib().orc_vision_linear(qtype, ptr(W), ptr(S), ptr(bias_bits), m, K, N, act, 0, ptr(x_bits), ptr(out),
                                       None, None) == 1
        return out
    outs = [np.zeros((m, split), np.uint16) for _ in range(3)]
    assert lib().orc_vision_linear(qtype, ptr(W), ptr(S), ptr(bias_bits), m, K, N, act, split, ptr(x_bits),
                                   *[ptr(o) for o in outs]) == 1
    return tuple(outs)


def swiglu(qtype, G, Gs, U, Us, rows, K, x_bits) -> np.ndarray:
    mid = np.zeros(rows, np.uint16)
    assert lib().orc_swiglu_mid(qtype, ptr(G), ptr(Gs), ptr(U), ptr(Us), rows, K, ptr(x_bits), ptr(mid)) == 1
    return mid


def rmsnorm_f16(x_bits, w_bits, eps=1e-6) -> np.ndarray:
    out = np.zeros(x_bits.size, np.uint16)
    assert lib().orc_rmsnorm_f16(ptr(x_bits), ptr(w_bits), x_bits.size, eps, ptr(out)) == 1
    return out


def lm_head_argmax(qtype, W, S, vocab, K, x_bits) -> tuple[int, float, float]:
    i, s1, s2 = _I32(), _F(), _F()
    assert lib().orc_lm_head_argmax(qtype, ptr(W), ptr(S), vocab, K, ptr(x_bits), ct.byref(i), ct.byref(s1),
                                    ct.byref(s2)) == 1
    return i.value, s1.value, s2.value


def router_topk(x_bits, R_bits, n_experts=64, top_k=6, norm_topk=False):
    ids = np.zeros(top_k, np.uint32)
    w = np.zeros(top_k, np.float32)
    probs = np.zeros(n_experts, np.float32)
    margin = np.zeros(1, np.float32)
    assert lib().orc_router_topk(ptr(x_bits), ptr(R_bits), n_experts, x_bits.size, top_k, int(norm_topk), ptr(ids),
                                 ptr(w), ptr(probs), ptr(margin)) == 1
    return ids, w, probs, float(margin[0])


def attention_decode(q_bits, k_cache, v_cache, prompt_len, gen, capacity, heads=10, head_dim=128):
    """k/v caches in the reference layout [cache_token][heads][head_dim] (fp16 bits)."""
    plan = Plan()
    if gen == 0:
        plan.prompt_length = plan.attention_length = prompt_len
        plan.ring_window = 128
    else:
        assert lib().orc_decode_attention_plan(prompt_len, capacity, 128, gen, ct.byref(plan)) == 1
    out = np.zeros(heads * head_dim, np.uint16)
    assert lib().orc_attention_decode(ptr(q_bits), ptr(k_cache), ptr(v_cache), heads, head_dim, ct.byref(plan),
                                      ptr(out)) == 1
    return out


def rope_f16(q_bits, k_bits, position, heads=10, head_dim=128):
    q = q_bits.copy()
    k = k_bits.copy()
    assert lib().orc_rope_f16(ptr(q), ptr(k), heads, head_dim, position, 10000.0) == 1
    return q, k


def embed_row(qtype, W, S, rows, K, token) -> np.ndarray:
    out = np.zeros(K, np.uint16)
    assert lib().orc_embed_row(qtype, ptr(W), ptr(S), rows, K, token, ptr(out)) == 1
    return out


class Model:
    """Oracle view of a .uocr image held in memory (numpy uint8 array or raw pointer + size)."""

    def __init__(self, data_ptr: int, size: int, keepalive=None, prompt_capacity: int = 1024) -> None:
        err = ct.create_string_buffer(256)
        self._keep = keepalive
        self.h = lib().orc_model_open(ct.c_void_p(data_ptr), size, err, 256)
        if not self.h:
            raise RuntimeError(f"oracle model open failed: {err.value.decode()}")
        self.s = lib().orc_session_create(ct.c_void_p(self.h), prompt_capacity)
        if not self.s:
            raise MemoryError("oracle session")

    def generate(self, ids, mask=None, image_rows_bits=None, max_new=8, ignore_eos=False):
        ids = np.ascontiguousarray(ids, np.int32)
        m = None if mask is None else np.ascontiguousarray(mask, np.uint8)
        rows = None if image_rows_bits is None else np.ascontiguousarray(image_rows_bits, np.uint16)
        out = np.zeros(max_new, np.int32)
        margins = np.zeros(max_new, np.float32)
        n = lib().orc_generate(ct.c_void_p(self.s), ptr(ids), ptr(m), ptr(rows), ids.size, max_new, int(ignore_eos),
                               ptr(out), ptr(margins))
        if n < 0:
            raise RuntimeError("oracle generation failed")
        return out[:n], margins[:n]

    def embed(self, token: int, out: np.ndarray) -> int:
        """Embedding row of token into out (uint16 fp16 bits [1280]); 1 on success."""
        return lib().orc_session_embed(ct.c_void_p(self.s), int(token), ptr(out))

    def close(self) -> None:
        if self.s:
            lib().orc_session_destroy(ct.c_void_p(self.s))
            self.s = None
        if self.h:
            lib().orc_model_close(ct.c_void_p(self.h))
            self.h = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass
