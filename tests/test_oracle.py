"""Pins the CPU oracle before it is used as the checker.

Each oracle function is checked against something other than its own
formula: the reference's golden vectors (tests/fixtures/cpu_ref_tiny_golden.h,
carried over as tests/golden/cpu_ref_tiny_golden.json), the closed forms and
known answers of the reference's tests/test_cpu_ref.c, the reference's own
uocr_cpu_ref.c compiled from its source (oracle/_ref, when present), the
converter's quantisation algorithm (src/unlimitedocr_c/convert.py:2058-2063,
:2249-2276) and float64 brute force.
"""
from __future__ import annotations

import ctypes as ct
import json
import math
from pathlib import Path

import numpy as np
import pytest

from conftest import convert_q4, convert_q8, dequant, q4_weights, q8_weights, rand_f16

GOLDEN = json.loads((Path(__file__).parent / "golden" / "cpu_ref_tiny_golden.json").read_text())


def f32(a):
    return np.ascontiguousarray(a, np.float32)


def close(a, b, tol):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    assert a.shape == b.shape
    assert np.all(np.abs(a - b) <= tol * np.maximum(1.0, np.abs(b))), (a, b)


# ---------------------------------------------------------------------------
# golden vectors (test_cpu_ref.c:509-607 tolerances)
# ---------------------------------------------------------------------------

def test_golden_rmsnorm(oracle):
    g = GOLDEN
    x, w = f32(g["UOCR_TINY_RMS_INPUT"]), f32(g["UOCR_TINY_RMS_WEIGHT"])
    out = np.zeros_like(x)
    assert oracle.lib().orc_rmsnorm_f32(x.ctypes.data, w.ctypes.data, g["UOCR_TINY_RMS_ROWS"], g["UOCR_TINY_RMS_COLS"],
                                        g["UOCR_TINY_RMS_EPS"], out.ctypes.data) == 1
    close(out, g["UOCR_TINY_RMS_EXPECTED"], 1e-5)


def test_golden_rope(oracle):
    g = GOLDEN
    q, k = f32(g["UOCR_TINY_ROPE_Q"]), f32(g["UOCR_TINY_ROPE_K"])
    qo, ko = np.zeros_like(q), np.zeros_like(k)
    assert oracle.lib().orc_rope_split_half_f32(q.ctypes.data, k.ctypes.data, g["UOCR_TINY_ROPE_TOKENS"],
                                                g["UOCR_TINY_ROPE_HEADS"], g["UOCR_TINY_ROPE_HEAD_DIM"],
                                                g["UOCR_TINY_ROPE_START"], g["UOCR_TINY_ROPE_THETA"], qo.ctypes.data,
                                                ko.ctypes.data) == 1
    close(qo, g["UOCR_TINY_ROPE_EXPECTED_Q"], 2e-5)
    close(ko, g["UOCR_TINY_ROPE_EXPECTED_K"], 2e-5)


def test_golden_sdpa(oracle):
    g = GOLDEN
    q, k, v = f32(g["UOCR_TINY_SDPA_Q"]), f32(g["UOCR_TINY_SDPA_K"]), f32(g["UOCR_TINY_SDPA_V"])
    out = np.zeros_like(q)
    assert oracle.lib().orc_causal_sdpa_f32(q.ctypes.data, k.ctypes.data, v.ctypes.data, g["UOCR_TINY_SDPA_TOKENS"],
                                            g["UOCR_TINY_SDPA_HEADS"], g["UOCR_TINY_SDPA_HEAD_DIM"],
                                            g["UOCR_TINY_SDPA_SCALE"], out.ctypes.data) == 1
    close(out, g["UOCR_TINY_SDPA_EXPECTED"], 2e-5)


def test_golden_swiglu(oracle):
    g = GOLDEN
    x = f32(g["UOCR_TINY_SWIGLU_INPUT"])
    ws = np.zeros(g["UOCR_TINY_SWIGLU_WORKSPACE_COUNT"], np.float32)
    out = np.zeros(g["UOCR_TINY_SWIGLU_INPUT_COUNT"], np.float32)
    args = [f32(g[k]) for k in ("UOCR_TINY_SWIGLU_GATE", "UOCR_TINY_SWIGLU_UP", "UOCR_TINY_SWIGLU_DOWN")]
    assert oracle.lib().orc_dense_swiglu_f32(x.ctypes.data, *[a.ctypes.data for a in args], g["UOCR_TINY_SWIGLU_ROWS"],
                                             g["UOCR_TINY_SWIGLU_HIDDEN"], g["UOCR_TINY_SWIGLU_INTERMEDIATE"],
                                             ws.ctypes.data, out.ctypes.data) == 1
    close(ws, g["UOCR_TINY_SWIGLU_EXPECTED_WORKSPACE"], 2e-5)
    close(out, g["UOCR_TINY_SWIGLU_EXPECTED"], 2e-5)


def test_golden_moe_router_and_experts(oracle):
    g = GOLDEN
    rows, e, k = g["UOCR_TINY_MOE_ROWS"], g["UOCR_TINY_MOE_EXPERTS"], g["UOCR_TINY_MOE_TOPK"]
    arrays = [f32(g[n]) for n in ("UOCR_TINY_MOE_INPUT", "UOCR_TINY_MOE_ROUTER", "UOCR_TINY_MOE_EXPERT_GATE",
                                  "UOCR_TINY_MOE_EXPERT_UP", "UOCR_TINY_MOE_EXPERT_DOWN", "UOCR_TINY_MOE_SHARED_GATE",
                                  "UOCR_TINY_MOE_SHARED_UP", "UOCR_TINY_MOE_SHARED_DOWN")]
    logits = np.zeros(rows * e, np.float32)
    probs = np.zeros(rows * e, np.float32)
    ids = np.zeros(rows * k, np.uint32)
    wts = np.zeros(rows * k, np.float32)
    ews = np.zeros(g["UOCR_TINY_MOE_EXPERT_WORKSPACE_COUNT"], np.float32)
    sws = np.zeros(g["UOCR_TINY_MOE_SHARED_WORKSPACE_COUNT"], np.float32)
    out = np.zeros(g["UOCR_TINY_MOE_INPUT_COUNT"], np.float32)
    assert oracle.lib().orc_moe_swiglu_f32(*[a.ctypes.data for a in arrays], rows, g["UOCR_TINY_MOE_HIDDEN"], e, k,
                                           g["UOCR_TINY_MOE_EXPERT_INTERMEDIATE"],
                                           g["UOCR_TINY_MOE_SHARED_INTERMEDIATE"], g["UOCR_TINY_MOE_SCALING"],
                                           logits.ctypes.data, probs.ctypes.data, ids.ctypes.data, wts.ctypes.data,
                                           ews.ctypes.data, sws.ctypes.data, out.ctypes.data) == 1
    close(logits, g["UOCR_TINY_MOE_EXPECTED_LOGITS"], 2e-5)
    close(probs, g["UOCR_TINY_MOE_EXPECTED_PROBS"], 2e-5)
    assert ids.tolist() == g["UOCR_TINY_MOE_EXPECTED_TOP_IDS"]
    close(wts, g["UOCR_TINY_MOE_EXPECTED_TOP_WEIGHTS"], 2e-5)
    close(ews, g["UOCR_TINY_MOE_EXPECTED_EXPERT_WORKSPACE"], 3e-5)
    close(sws, g["UOCR_TINY_MOE_EXPECTED_SHARED_WORKSPACE"], 3e-5)
    close(out, g["UOCR_TINY_MOE_EXPECTED"], 3e-5)
    # raw (un-renormalised) top-6 probabilities: they do not sum to 1
    assert float(np.sum(wts[:k])) < 1.0


# ---------------------------------------------------------------------------
# known answers / closed forms of test_cpu_ref.c
# ---------------------------------------------------------------------------

def test_f16_known_answers(oracle):
    L = oracle.lib()
    assert L.orc_bf16_to_f32(0x3F80) == 1.0 and L.orc_bf16_to_f32(0xC020) == -2.5
    assert L.orc_f16_to_f32(0x3C00) == 1.0 and L.orc_f16_to_f32(0xC000) == -2.0
    assert L.orc_f32_to_f16(0.0) == 0x0000 and L.orc_f32_to_f16(-0.0) == 0x8000
    assert L.orc_f32_to_f16(1.0) == 0x3C00 and L.orc_f32_to_f16(-2.0) == 0xC000
    assert L.orc_f32_to_f16(65504.0) == 0x7BFF and L.orc_f32_to_f16(math.inf) == 0x7C00
    assert (L.orc_f32_to_f16(math.nan) & 0x7C00) == 0x7C00
    assert L.orc_f32_to_f16(0.5) == 0x3800


def test_f16_conversion_matches_numpy_exhaustively(oracle):
    """numpy's float16 is IEEE binary16 with round-to-nearest-even."""
    L = oracle.lib()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = np.array([L.orc_f16_to_f32(int(b)) for b in bits[::7]], np.float32)
    ref = bits[::7].view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(ours[finite], ref[finite]) and np.all(np.isnan(ours[~finite]) == np.isnan(ref[~finite]))
    rng = np.random.default_rng(3)
    xs = np.concatenate([rng.standard_normal(4000).astype(np.float32) * s for s in (1e-7, 1e-5, 1e-3, 1, 1e3, 3e4)])
    ours = np.array([L.orc_f32_to_f16(float(x)) for x in xs], np.uint16)
    assert np.array_equal(ours, xs.astype(np.float16).view(np.uint16))


def test_rmsnorm_closed_form(oracle):
    x = f32([1, 2, 3, 4, 0, -1, 1, 0.5])
    w = f32([1, 0.5, -1, 2])
    out = np.zeros_like(x)
    assert oracle.lib().orc_rmsnorm_f32(x.ctypes.data, w.ctypes.data, 2, 4, 1e-6, out.ctypes.data) == 1
    r = x.reshape(2, 4).astype(np.float64)
    exp = r / np.sqrt((r * r).mean(1, keepdims=True) + 1e-6) * w
    close(out.reshape(2, 4), exp, 1e-6)
    assert oracle.lib().orc_rmsnorm_f32(x.ctypes.data, w.ctypes.data, 2, 4, -1.0, out.ctypes.data) == 0


def test_rope_closed_form(oracle):
    q = f32([1, 2, 3, 4, 1, 2, 3, 4])
    k = -q
    qo, ko = np.zeros_like(q), np.zeros_like(k)
    assert oracle.lib().orc_rope_split_half_f32(q.ctypes.data, k.ctypes.data, 2, 1, 4, 0, 10000.0, qo.ctypes.data,
                                                ko.ctypes.data) == 1
    assert np.array_equal(qo[:4], q[:4]) and np.array_equal(ko[:4], k[:4])
    c0, s0, c1, s1 = math.cos(1), math.sin(1), math.cos(0.01), math.sin(0.01)
    close(qo[4:], [1 * c0 - 3 * s0, 2 * c1 - 4 * s1, 3 * c0 + 1 * s0, 4 * c1 + 2 * s1], 1e-6)
    assert oracle.lib().orc_rope_split_half_f32(q.ctypes.data, k.ctypes.data, 2, 1, 3, 0, 10000.0, qo.ctypes.data,
                                                ko.ctypes.data) == 0


def test_router_ties_go_to_lower_id(oracle):
    x = f32([0, 0])
    r = f32([1, 0, 0, 1, 1, 1, -1, 0])
    logits, probs = np.zeros(4, np.float32), np.zeros(4, np.float32)
    ids, w = np.zeros(2, np.uint32), np.zeros(2, np.float32)
    assert oracle.lib().orc_moe_router_f32(x.ctypes.data, r.ctypes.data, 1, 2, 4, 2, 1.0, logits.ctypes.data,
                                           probs.ctypes.data, ids.ctypes.data, w.ctypes.data) == 1
    assert ids.tolist() == [0, 1]
    close(w, [0.25, 0.25], 1e-6)
    assert oracle.lib().orc_moe_router_f32(x.ctypes.data, r.ctypes.data, 1, 2, 4, 5, 1.0, logits.ctypes.data,
                                           probs.ctypes.data, ids.ctypes.data, w.ctypes.data) == 0


def test_kv_ring_known_answers(oracle):
    """test_cpu_ref.c:627-708: prompt capacity 4, ring 3, prompt length 3."""
    L = oracle.lib()
    out = ct.c_uint32()
    expect = {0: 0, 2: 2, 3: 3, 4: 4, 5: 5, 6: 3}
    for pos, tok in expect.items():
        assert L.orc_kv_cache_token_for_position(3, 4, 3, pos, ct.byref(out)) == 1 and out.value == tok
    assert L.orc_kv_cache_token_for_position(5, 4, 3, 0, ct.byref(out)) == 0
    plan = oracle.Plan()
    assert L.orc_decode_attention_plan(3, 4, 3, 5, ct.byref(plan)) == 1
    assert (plan.generated_count, plan.live_generated, plan.first_generated_index, plan.query_position,
            plan.attention_length) == (5, 3, 2, 7, 6)
    toks = []
    for i in range(plan.attention_length):
        assert L.orc_attention_index_to_token(ct.byref(plan), i, ct.byref(out)) == 1
        toks.append(out.value)
    assert toks == [0, 1, 2, 5, 3, 4]
    assert L.orc_attention_index_to_token(ct.byref(plan), plan.attention_length, ct.byref(out)) == 0
    assert L.orc_decode_attention_plan(3, 4, 3, 0, ct.byref(plan)) == 1
    assert (plan.live_generated, plan.attention_length, plan.query_position) == (0, 3, 3)


# ---------------------------------------------------------------------------
# the reference's own CPU path, built from its source
# ---------------------------------------------------------------------------

def test_against_reference_cpu_ref_build(oracle):
    ref = oracle.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    L = oracle.lib()
    ref.uocr_cpu_ref_f32_to_f16_bits.argtypes = [ct.c_float]
    ref.uocr_cpu_ref_f32_to_f16_bits.restype = ct.c_uint16
    ref.uocr_cpu_ref_f16_bits_to_f32.argtypes = [ct.c_uint16]
    ref.uocr_cpu_ref_f16_bits_to_f32.restype = ct.c_float
    rng = np.random.default_rng(11)
    for x in np.concatenate([rng.standard_normal(3000) * s for s in (1e-6, 1e-4, 1, 3e4)]).astype(np.float32):
        assert L.orc_f32_to_f16(float(x)) == ref.uocr_cpu_ref_f32_to_f16_bits(float(x))
    for b in range(0, 65536, 13):
        a, r = L.orc_f16_to_f32(b), ref.uocr_cpu_ref_f16_bits_to_f32(b)
        assert a == r or (math.isnan(a) and math.isnan(r))
    # fp32 ops on random shapes: identical arithmetic, identical results
    rows, hid, exp_n, topk, ei, si = 3, 16, 9, 4, 5, 6
    x = rng.standard_normal(rows * hid).astype(np.float32)
    w = rng.standard_normal(hid).astype(np.float32)
    a, b = np.zeros_like(x), np.zeros_like(x)
    assert L.orc_rmsnorm_f32(x.ctypes.data, w.ctypes.data, rows, hid, ct.c_float(1e-6), a.ctypes.data) == 1
    assert ref.uocr_cpu_ref_rmsnorm_f32(ct.c_void_p(x.ctypes.data), ct.c_void_p(w.ctypes.data), rows, hid,
                                        ct.c_float(1e-6), ct.c_void_p(b.ctypes.data)) == 1
    assert np.array_equal(a, b)
    mats = [rng.standard_normal(n).astype(np.float32) for n in
            (exp_n * hid, exp_n * ei * hid, exp_n * ei * hid, exp_n * hid * ei, si * hid, si * hid, hid * si)]
    outs = []
    for fn in (L.orc_moe_swiglu_f32, ref.uocr_cpu_ref_moe_swiglu_f32):
        bufs = [np.zeros(n, np.float32) for n in (rows * exp_n, rows * exp_n)] + [np.zeros(rows * topk, np.uint32)] + \
               [np.zeros(n, np.float32) for n in (rows * topk, rows * topk * ei, rows * si, rows * hid)]
        args = [ct.c_void_p(x.ctypes.data)] + [ct.c_void_p(m.ctypes.data) for m in mats] + \
               [rows, hid, exp_n, topk, ei, si, ct.c_float(1.0)] + [ct.c_void_p(q.ctypes.data) for q in bufs]
        assert fn(*args) == 1
        outs.append(bufs)
    for p, q in zip(*outs):
        assert np.array_equal(p, q)


# ---------------------------------------------------------------------------
# quantised formats: the converter's algorithm, restated from convert.py
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("qtype", [3, 4])
def test_weight_storage_matches_converter(oracle, qtype):
    rng = np.random.default_rng(5)
    vals = (rng.standard_normal((8, 256)) * 0.05).astype(np.float32)
    vals[2, 64:128] = 0.0  # all-zero group
    if qtype == 3:
        w, s = convert_q8(vals)
        deq = w.astype(np.float32).reshape(8, 4, 64) * s.astype(np.float32)[:, :, None]
        deq = deq.reshape(8, 256)
    else:
        w, s, deq = convert_q4(vals)
    ours = np.array([[oracle.lib().orc_weight_at(qtype, w.ctypes.data, s.ctypes.data, 256, r, c) for c in range(256)]
                     for r in range(8)], np.float32)
    assert np.array_equal(ours, deq)
    assert np.all(ours[2, 64:128] == 0.0)
    # Q8: |err| <= scale/2 plus up to 127 fp16 rounding steps of the stored
    # scale (quantised with the fp32 scale).  Q4: the group's signed max maps
    # to -8 exactly, so values of the opposite sign near the max clip at +7,
    # an error of up to one step.
    slack = 1.0 if qtype == 4 else 0.5 + 127 * 2.0 ** -11
    step = np.repeat(np.abs(s.astype(np.float32)), 64, axis=1) * slack * 1.0001
    assert np.all(np.abs(ours - vals) <= step + 1e-7)


@pytest.mark.parametrize("qtype", [1, 3, 4])
def test_row_dot_vs_float64(oracle, qtype):
    rng = np.random.default_rng(qtype)
    rows, k = 6, 1280
    w, s = {1: lambda: (rand_f16(rng, (rows, k), 0.01), None), 3: lambda: q8_weights(rng, rows, k),
            4: lambda: q4_weights(rng, rows, k)}[qtype]()
    x = rand_f16(rng, k)
    ref = dequant(qtype, w, s).astype(np.float64) @ x.astype(np.float64)
    xb = x.view(np.uint16)
    got = [oracle.lib().orc_row_dot(qtype, w.ctypes.data, None if s is None else s.ctypes.data, k, r, xb.ctypes.data)
           for r in range(rows)]
    assert np.allclose(got, ref, rtol=1e-4, atol=1e-5)
    y = oracle.gemv(qtype, w, s, rows, k, xb)
    assert np.allclose(y.view(np.float16).astype(np.float64), ref, rtol=2e-3, atol=1e-3)


def test_lm_head_argmax_rules(oracle):
    rng = np.random.default_rng(9)
    vocab, k = 300, 1280
    w, s = q4_weights(rng, vocab, k)
    w[200] = w[57]  # exact duplicate row -> tie, lower id must win
    s[200] = s[57]
    x = rand_f16(rng, k)
    scores = dequant(4, w, s).astype(np.float64) @ x.astype(np.float64)
    best = int(np.argmax(scores))
    w[57] = w[best]
    s[57] = s[best]
    w[200] = w[best]
    s[200] = s[best]
    tid, s1, s2 = oracle.lm_head_argmax(4, w, s, vocab, k, x.view(np.uint16))
    assert tid == min(57, best)
    # NaN rows are skipped (a NaN scale makes the whole row NaN)
    s_nan = s.copy()
    s_nan[min(57, best), 0] = np.float16(np.nan)
    s_nan[200, 0] = np.float16(np.nan)
    s_nan[max(57, best), 0] = np.float16(np.nan)
    tid2, _, _ = oracle.lm_head_argmax(4, w, s_nan, vocab, k, x.view(np.uint16))
    scores[[57, 200, best]] = -np.inf
    assert tid2 == int(np.argmax(scores))
    # no valid row -> id 0
    all_nan = np.full_like(s, np.float16(np.nan))
    tid3, score3, _ = oracle.lm_head_argmax(4, w, all_nan, vocab, k, x.view(np.uint16))
    assert tid3 == 0 and score3 == -np.inf


def test_router_vs_sort(oracle):
    rng = np.random.default_rng(4)
    x = rand_f16(rng, 1280)
    r = rand_f16(rng, (64, 1280), 0.03)
    ids, w, probs, margin = oracle.router_topk(x.view(np.uint16), r.view(np.uint16))
    logits = r.astype(np.float64) @ x.astype(np.float64)
    p = np.exp(logits - logits.max())
    p /= p.sum()
    order = np.lexsort((np.arange(64), -p))[:6]
    assert ids.tolist() == order.tolist()
    assert np.allclose(w, p[order], rtol=1e-4)
    ids2, w2, _, _ = oracle.router_topk(x.view(np.uint16), r.view(np.uint16), norm_topk=True)
    assert ids2.tolist() == ids.tolist() and abs(float(w2.sum()) - 1.0) < 1e-5


def test_attention_decode_ring_vs_float64(oracle):
    rng = np.random.default_rng(2)
    heads, hd, prompt, cap, gen = 10, 128, 40, 40 + 128, 150
    kc = rand_f16(rng, (cap, heads, hd))
    vc = rand_f16(rng, (cap, heads, hd))
    q = rand_f16(rng, heads * hd)
    out = oracle.attention_decode(q.view(np.uint16), kc.view(np.uint16), vc.view(np.uint16), prompt, gen, prompt)
    live = min(gen, 128)
    first = gen - live
    slots = list(range(prompt)) + [prompt + (first + i) % 128 for i in range(live)]
    qf = q.astype(np.float64).reshape(heads, hd)
    ref = np.zeros((heads, hd))
    for h in range(heads):
        sc = kc[slots, h, :].astype(np.float64) @ qf[h] / math.sqrt(hd)
        p = np.exp(sc - sc.max())
        ref[h] = (p / p.sum()) @ vc[slots, h, :].astype(np.float64)
    assert np.allclose(out.view(np.float16).astype(np.float64).reshape(heads, hd), ref, atol=2e-3, rtol=2e-3)


def test_rope_f16_vs_float64(oracle):
    rng = np.random.default_rng(8)
    q, k = rand_f16(rng, 1280), rand_f16(rng, 1280)
    pos = 1037
    qo, ko = oracle.rope_f16(q.view(np.uint16), k.view(np.uint16), pos)
    d = np.arange(64)
    ang = pos * (10000.0 ** (-2.0 * d / 128))
    for src, got in ((q, qo), (k, ko)):
        x = src.astype(np.float64).reshape(10, 128)
        a, b = x[:, :64], x[:, 64:]
        exp = np.concatenate([a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)], axis=1)
        assert np.allclose(got.view(np.float16).astype(np.float64).reshape(10, 128), exp, atol=4e-3, rtol=2e-3)


def test_rmsnorm_f16_and_embed(oracle):
    rng = np.random.default_rng(12)
    x, w = rand_f16(rng, 1280), (rng.uniform(0.8, 1.2, 1280)).astype(np.float16)
    y = oracle.rmsnorm_f16(x.view(np.uint16), w.view(np.uint16))
    xf = x.astype(np.float64)
    exp = xf / np.sqrt(np.mean(xf * xf) + 1e-6) * w.astype(np.float64)
    assert np.allclose(y.view(np.float16).astype(np.float64), exp, rtol=1e-3, atol=1e-3)
    for qt in (1, 3, 4):
        W, S = {1: (rand_f16(rng, (20, 1280), 0.01), None), 3: q8_weights(rng, 20, 1280),
                4: q4_weights(rng, 20, 1280)}[qt]
        row = oracle.embed_row(qt, W, S, 20, 1280, 13)
        assert np.array_equal(row.view(np.float16), dequant(qt, W, S)[13].astype(np.float16))
        assert not oracle.embed_row(qt, W, S, 20, 1280, 20).any()  # out of range -> zeros


# ---------------------------------------------------------------------------
# vision linear (gemm_q8.metal:161-221, gemm_q4.metal:63-131, MPS fp16 path)
# ---------------------------------------------------------------------------

def _vision_float64(qtype, w, s, bias, x, act):
    """float64 brute force: weights staged as fp16(q * scale), the fp16 path's
    product rounded to fp16 (MPS), exact erf from scipy."""
    from scipy.special import erf

    from conftest import dequant
    wd = dequant(qtype, w, s).astype(np.float16).astype(np.float64)
    z = x.astype(np.float64) @ wd.T
    if qtype == 1:
        z = z.astype(np.float16).astype(np.float64)
    z = z + bias.astype(np.float64)
    if act == 1:
        z = z / (1.0 + np.exp(-1.702 * z))
    elif act == 2:
        z = 0.5 * z * (1.0 + erf(z / math.sqrt(2.0)))
    return z


@pytest.mark.parametrize("qtype", [1, 3, 4])
@pytest.mark.parametrize("act", [0, 1, 2])
def test_vision_linear_vs_float64(oracle, qtype, act):
    from conftest import weights_for
    rng = np.random.default_rng(10 * qtype + act)
    m, k, n = 5, 192, 48
    w, s = weights_for(qtype, rng, n, k)
    x = rand_f16(rng, (m, k))
    bias = rand_f16(rng, n, 2.0)  # spreads the pre-activations over the curved part of both GELUs
    got = oracle.vision_linear(qtype, w, s, bias.view(np.uint16), m, k, n, act, 0, x.view(np.uint16))
    got = got.view(np.float16).astype(np.float64)
    ref = _vision_float64(qtype, w, s, bias, x, act)
    # fp16 half-ulp of the output (4.9e-4 relative) plus fp32 accumulation and,
    # for the fp16 path, one product ulp when the two sums round differently
    assert np.all(np.abs(got - ref) <= 1e-3 * np.abs(ref) + 5e-4), np.abs(got - ref).max()


def test_vision_linear_split_is_column_thirds(oracle):
    rng = np.random.default_rng(77)
    m, k, split = 7, 128, 64
    w, s = q8_weights(rng, 3 * split, k)
    x = rand_f16(rng, (m, k)).view(np.uint16)
    bias = rand_f16(rng, 3 * split).view(np.uint16)
    whole = oracle.vision_linear(3, w, s, bias, m, k, 3 * split, 0, 0, x)
    q, kk, v = oracle.vision_linear(3, w, s, bias, m, k, 3 * split, 0, split, x)
    assert np.array_equal(np.hstack([q, kk, v]), whole)


def test_vision_linear_rejects(oracle):
    lib = oracle.lib()
    p = oracle.ptr
    w = np.zeros((96, 128), np.int8)
    s = np.ones((96, 2), np.float16)
    b = np.zeros(96, np.uint16)
    x = np.zeros((2, 128), np.uint16)
    o = np.zeros((2, 96), np.uint16)
    assert lib.orc_vision_linear(3, p(w), p(s), p(b), 2, 128, 96, 0, 0, p(x), p(o), None, None) == 1
    assert lib.orc_vision_linear(3, p(w), p(s), p(b), 2, 100, 96, 0, 0, p(x), p(o), None, None) == 0  # k % 64
    assert lib.orc_vision_linear(3, p(w), p(s), None, 2, 128, 96, 0, 0, p(x), p(o), None, None) == 0  # bias
    assert lib.orc_vision_linear(3, p(w), p(s), p(b), 2, 128, 96, 3, 0, p(x), p(o), None, None) == 0  # act
    assert lib.orc_vision_linear(3, p(w), p(s), p(b), 2, 128, 96, 0, 30, p(x), p(o), p(o), p(o)) == 0  # n != 3 split
