"""Pins of the oracle's compositions against the reference's own CPU ops.

`orc_forward_token` (one decode step through the 12 layers) and
`orc_moe_ffn` (one MoE FFN) are compositions of individually pinned pieces.
Here the same computation is rebuilt independently from the reference's
compiled CPU path (`oracle/_ref`, built from src/backend/cpu_ref/uocr_cpu_ref.c:
rmsnorm :145, rope :171, causal sdpa :227, dense swiglu :305, moe swiglu
:468) plus numpy matrix-vector products for the projections, wired in the
reference's decode order (uocr_metal.m:14299-14518) with fp16 storage at
the golden.py:381-666 rounding points.  A dropped residual, a swapped norm,
a wrong RoPE position or a misplaced expert stride shows up as a large
difference; fp32 summation order and the reference ops' unrounded
intermediates (the SwiGLU mid and the shared-expert output stay fp32
there) account for the small one.

Skipped when the reference tree (and so `oracle/_ref`) is absent, e.g. on
the GPU box.
"""
from __future__ import annotations

import ctypes as ct

import numpy as np
import pytest

H, NH, HD, L = 1280, 10, 128, 12
E, K, EI, SI, I0 = 64, 6, 896, 1792, 6848
F = ct.c_float


def _p(a):
    return ct.c_void_p(a.ctypes.data)


@pytest.fixture(scope="module")
def ref(oracle):
    lib = oracle.ref_lib()
    if lib is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    return lib


@pytest.fixture(scope="module")
def f16_model(uocr):
    m = uocr.synth_model(uocr.QPROFILE_FP16, 11)
    yield m
    m.close()


class Weights:
    """fp32 copies of one layer's tensors from an fp16 .uocr image."""

    def __init__(self, uocr, image, table):
        self.uocr, self.image = uocr, image
        self.by_id = {int(e["id"]): e for e in table}

    def get(self, tid, rows, cols):
        return self.uocr.f16_tensor(self.image, self.by_id[tid], rows, cols).astype(np.float32)

    def vec(self, tid, n):
        return self.get(tid, 1, n)[0]

    def layer(self, l):
        b = 10000 + 1000 * l
        d = dict(in_norm=self.vec(b + 1, H), post_norm=self.vec(b + 2, H),
                 q=self.get(b + 10, H, H), k=self.get(b + 11, H, H), v=self.get(b + 12, H, H),
                 o=self.get(b + 13, H, H))
        if l == 0:
            d.update(gate=self.get(b + 30, I0, H), up=self.get(b + 31, I0, H), down=self.get(b + 32, H, I0))
        else:
            d.update(router=self.get(b + 40, E, H), sg=self.get(b + 50, SI, H), su=self.get(b + 51, SI, H),
                     sd=self.get(b + 52, H, SI),
                     eg=np.stack([self.get(b + 100 + 3 * e, EI, H) for e in range(E)]),
                     eu=np.stack([self.get(b + 101 + 3 * e, EI, H) for e in range(E)]),
                     ed=np.stack([self.get(b + 102 + 3 * e, H, EI) for e in range(E)]))
        return d


def f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def ref_rmsnorm(ref, x, w):
    out = np.zeros(H, np.float32)
    assert ref.uocr_cpu_ref_rmsnorm_f32(_p(x), _p(w), 1, H, F(1e-6), _p(out)) == 1
    return out


def ref_rope(ref, q, k, pos):
    qo, ko = np.zeros(H, np.float32), np.zeros(H, np.float32)
    assert ref.uocr_cpu_ref_rope_split_half_f32(_p(q), _p(k), 1, NH, HD, pos, F(10000.0), _p(qo), _p(ko)) == 1
    return qo, ko


def ref_attention(ref, q, Ks, Vs):
    """Last query row of the reference's causal SDPA over positions 0..t."""
    n = len(Ks)
    Q = np.zeros((n, H), np.float32)
    Q[-1] = q
    Kc, Vc = np.ascontiguousarray(np.stack(Ks)), np.ascontiguousarray(np.stack(Vs))
    out = np.zeros((n, H), np.float32)
    assert ref.uocr_cpu_ref_causal_sdpa_f32(_p(Q), _p(Kc), _p(Vc), n, NH, HD, F(1.0 / np.sqrt(HD)), _p(out)) == 1
    return out[-1]


def ref_dense(ref, x, w):
    ws, out = np.zeros(I0, np.float32), np.zeros(H, np.float32)
    assert ref.uocr_cpu_ref_dense_swiglu_f32(_p(x), _p(w["gate"]), _p(w["up"]), _p(w["down"]), 1, H, I0, _p(ws),
                                             _p(out)) == 1
    return out


def ref_moe(ref, x, w):
    logits, probs = np.zeros(E, np.float32), np.zeros(E, np.float32)
    ids, tw = np.zeros(K, np.uint32), np.zeros(K, np.float32)
    ews, sws, out = np.zeros(K * EI, np.float32), np.zeros(SI, np.float32), np.zeros(H, np.float32)
    assert ref.uocr_cpu_ref_moe_swiglu_f32(_p(x), _p(w["router"]), _p(w["eg"]), _p(w["eu"]), _p(w["ed"]), _p(w["sg"]),
                                           _p(w["su"]), _p(w["sd"]), 1, H, E, K, EI, SI, F(1.0), _p(logits),
                                           _p(probs), _p(ids), _p(tw), _p(ews), _p(sws), _p(out)) == 1
    srt = np.sort(logits)[::-1]
    margin = float(np.min(srt[:K] - srt[1:K + 1]))
    return out, ids, margin


def test_forward_token_matches_reference_ops(uocr, oracle, ref, f16_model):
    """Three prompt positions through all 12 layers: the oracle's
    orc_forward_token against the reference-op composition."""
    image = f16_model.view()
    W = Weights(uocr, image, uocr.tensor_table(image))
    T = 3
    rng = np.random.default_rng(4)
    h0 = rng.standard_normal((T, H)).astype(np.float16)

    # oracle: token-major
    orc = oracle.Model(f16_model.ptr, f16_model.size, f16_model, prompt_capacity=8)
    Lb = oracle.lib()
    assert Lb.orc_session_reset(ct.c_void_p(orc.s), T) == 1
    got = h0.view(np.uint16).copy()
    traces = np.zeros((T, (L - 1) * K), np.uint32)
    for t in range(T):
        assert Lb.orc_forward_token(ct.c_void_p(orc.s), got[t].ctypes.data, t, traces[t].ctypes.data) == 1
    orc.close()

    # reference ops: layer-major (identical under causal attention)
    h = h0.astype(np.float32)
    Ks, Vs = [[] for _ in range(L)], [[] for _ in range(L)]
    ids_checked = 0
    for l in range(L):
        w = W.layer(l)
        for t in range(T):
            n = f16(ref_rmsnorm(ref, h[t], w["in_norm"]))
            q, k, v = f16(w["q"] @ n), f16(w["k"] @ n), f16(w["v"] @ n)
            q, k = ref_rope(ref, q, k, t)
            q, k = f16(q), f16(k)
            Ks[l].append(k)
            Vs[l].append(v)
            ctx = f16(ref_attention(ref, q, Ks[l], Vs[l]))
            a = f16(w["o"] @ ctx + h[t])
            n2 = f16(ref_rmsnorm(ref, a, w["post_norm"]))
            if l == 0:
                h[t] = f16(ref_dense(ref, n2, w) + a)
            else:
                out, ids, margin = ref_moe(ref, n2, w)
                if margin > 1e-2:
                    assert traces[t][(l - 1) * K:l * K].tolist() == ids.tolist(), f"layer {l} position {t}"
                    ids_checked += 1
                h[t] = f16(out + a)
    gotf = got.view(np.float16).astype(np.float64)
    err = np.abs(gotf - h)
    tol = 2e-2 + 1e-2 * np.abs(h)
    assert np.all(err <= tol), f"max err {err.max()} (value {h.flat[int(err.argmax())]})"
    assert ids_checked >= 10


def test_moe_ffn_matches_reference_op(uocr, oracle, ref, f16_model):
    """orc_moe_ffn (router, shared + 6 routed experts, combine) on layer 1's
    fp16 weights against the reference's moe swiglu + residual."""
    image = f16_model.view()
    W = Weights(uocr, image, uocr.tensor_table(image))
    w = W.layer(1)
    table = {int(e["id"]): e for e in uocr.tensor_table(image)}
    b = 11000

    def raw(tid):
        e = table[tid]
        off = int(e["payload_offset"])
        return image[off:off + int(e["payload_size"])]

    ev = oracle.ExpertView()
    ev.qtype = 1
    ev.gate_w, ev.up_w, ev.down_w = (raw(b + 100 + j).ctypes.data for j in range(3))
    ev.gate_s = ev.up_s = ev.down_s = None
    ev.w_stride = int(table[b + 103]["payload_offset"]) - int(table[b + 100]["payload_offset"])
    ev.s_stride = 0
    rng = np.random.default_rng(6)
    checked = 0
    for _ in range(24):
        x = f16(ref_rmsnorm(ref, rng.standard_normal(H).astype(np.float32), w["post_norm"]))
        res = rng.standard_normal(H).astype(np.float16)
        xb, rb = x.astype(np.float16).view(np.uint16), res.view(np.uint16)
        out = np.zeros(H, np.uint16)
        ids, wts, margin = np.zeros(K, np.uint32), np.zeros(K, np.float32), np.zeros(1, np.float32)
        assert oracle.lib().orc_moe_ffn(_p(xb), _p(rb), raw(b + 40).ctypes.data, E, K, 0, ct.byref(ev), EI, 1,
                                        raw(b + 50).ctypes.data, None, raw(b + 51).ctypes.data, None,
                                        raw(b + 52).ctypes.data, None, SI, _p(out), _p(ids), _p(wts),
                                        _p(margin)) == 1
        rout, rids, rmargin = ref_moe(ref, x, w)
        if rmargin > 1e-2:
            assert ids.tolist() == rids.tolist()
            expect = f16(rout + res.astype(np.float32))
            got = out.view(np.float16).astype(np.float64)
            assert np.all(np.abs(got - expect) <= 2e-2 + 1e-2 * np.abs(expect))
            checked += 1
    assert checked >= 3
