"""GPU parity of the MFMA prefill operators and the engine's batched prefill.

The prefill processes all prompt rows of a layer at once (tiled MFMA GEMMs,
causal flash attention, bucketed MoE).  Every row it produces must match the
oracle's per-row decode arithmetic within the BASELINE tolerance (fp16
max-abs 2e-2 / rel 1e-2); expert and token ids bit-exact where the oracle's
margin exceeds 1e-2.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rand_f16, weights_for
from test_gpu_ops import _moe_setup, _oracle_moe, assert_f16_close, dev, to_ref_layout
from test_gpu_engine import compare_ids, model, prompt

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("qtype,m,n,k", [(4, 37, 1280, 1280), (3, 65, 3840, 1280), (1, 33, 896, 1792),
                                         (4, 20, 6848, 1280), (4, 9, 1280, 6848), (3, 130, 64, 1280),
                                         (4, 1, 1792, 1280), (3, 64, 1280, 896)])
def test_gemm_matches_oracle_rows(gpu, oracle, qtype, m, n, k):
    """Every output row equals the oracle GEMV of that row (with and without residual)."""
    uocr = gpu
    rng = np.random.default_rng(m * 7 + n + k + qtype)
    w, s = weights_for(qtype, rng, n, k)
    x = rand_f16(rng, (m, k))
    res = rand_f16(rng, (m, n))
    dw, ds = dev(uocr, w), None if s is None else dev(uocr, s)
    dx, dres, dy = dev(uocr, x), dev(uocr, res), uocr.DeviceBuffer(m * n * 2)
    for with_res in (False, True):
        uocr.op_gemm(qtype, dw, ds, m, n, k, dx, dres if with_res else None, dy)
        uocr.sync()
        got = dy.download(np.uint16).reshape(m, n)
        for r in range(m):
            ref = oracle.gemv(qtype, w, s, n, k, x[r].view(np.uint16), res[r].view(np.uint16) if with_res else None)
            assert_f16_close(got[r], ref)


def test_gemm_rejects_bad_shapes(gpu):
    uocr = gpu
    buf = uocr.DeviceBuffer(1 << 16)
    with pytest.raises(RuntimeError):
        uocr.op_gemm(4, buf, buf, 4, 128, 100, buf, None, buf)  # K not a multiple of 64
    with pytest.raises(RuntimeError):
        uocr.op_gemm(4, buf, None, 4, 128, 128, buf, None, buf)  # quantised weights need scales
    with pytest.raises(RuntimeError):
        uocr.op_gemm(2, buf, buf, 4, 128, 128, buf, None, buf)  # unsupported qtype


@pytest.mark.parametrize("P", [1, 63, 64, 150, 600, 932])
def test_prefill_attention_matches_oracle(gpu, oracle, P):
    """Causal attention: query i over slots 0..i equals the oracle's decode
    attention with prompt length i+1."""
    uocr = gpu
    rng = np.random.default_rng(P)
    cap = P + 128
    kc = rand_f16(rng, (10, cap, 128))
    vc = rand_f16(rng, (10, cap, 128))
    q = rand_f16(rng, (P, 1280))
    dctx = uocr.DeviceBuffer(P * 2560)
    uocr.op_prefill_attention(dev(uocr, q), dev(uocr, kc), dev(uocr, vc), cap, P, dctx)
    uocr.sync()
    got = dctx.download(np.uint16).reshape(P, 1280)
    kref, vref = to_ref_layout(kc).view(np.uint16), to_ref_layout(vc).view(np.uint16)
    for i in range(P):
        ref = oracle.attention_decode(q[i].view(np.uint16), kref, vref, i + 1, 0, P)
        assert_f16_close(got[i], ref, atol=5e-3, rtol=5e-3)


@pytest.mark.parametrize("qtype,shared_qtype", [(4, 4), (3, 3), (4, 3)])
def test_moe_ffn_rows_matches_oracle(gpu, oracle, qtype, shared_qtype):
    """Bucketed MoE over 48 rows: each row equals the oracle's single-token
    MoE FFN wherever the router margin exceeds 1e-2."""
    uocr = gpu
    rng = np.random.default_rng(77 + qtype + shared_qtype)
    m, host, keep = _moe_setup(uocr, rng, qtype, shared_qtype)
    P = 48
    nw = rng.uniform(0.8, 1.2, 1280).astype(np.float16)
    x = rand_f16(rng, (P, 1280))
    res = rand_f16(rng, (P, 1280))
    ws = uocr.moe_rows_workspace(P)
    dout = uocr.DeviceBuffer(P * 2560)
    uocr.op_moe_ffn_rows(m, dev(uocr, x), dev(uocr, nw), dev(uocr, res), P, 0, ws, dout)
    uocr.sync()
    got = dout.download(np.uint16).reshape(P, 1280)
    checked = 0
    for t in range(P):
        xn = oracle.rmsnorm_f16(x[t].view(np.uint16), nw.view(np.uint16))
        ref, _, _, margin = _oracle_moe(oracle, host, qtype, shared_qtype, xn, res[t].view(np.uint16))
        if margin > 1e-2:
            assert_f16_close(got[t], ref)
            checked += 1
    assert checked >= P // 4


@pytest.mark.parametrize("qprofile", [3, 2])
def test_batched_prefill_generation_matches_oracle(gpu, oracle, qprofile):
    """A 200-row prompt (4 GEMM row tiles, several rows per expert bucket)
    through the MFMA prefill, then greedy decode, against the oracle's
    position-by-position prefill."""
    uocr = gpu
    m = model(uocr, qprofile)
    eng = uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=256, max_gen_tokens=16)
    orc = oracle.Model(m.ptr, m.size, m, prompt_capacity=256)
    best = 0
    for seed in range(3):
        rng = np.random.default_rng(500 + 10 * qprofile + seed)
        ids, mask, rows = prompt(rng, 40, 160)
        got = eng.generate_embeddings(ids, mask, rows, 6, flags=uocr.GEN_IGNORE_EOS)[0]
        ref, margins = orc.generate(ids, mask, rows.view(np.uint16), max_new=6, ignore_eos=True)
        best = max(best, compare_ids(got.tolist(), ref.tolist(), margins.tolist()))
        if best >= 3:
            break
    orc.close()
    eng.close()
    assert best >= 3


def test_batched_and_token_prefill_agree(gpu):
    """The MFMA prefill and the per-position prefill leave the same hidden
    state for the first selection: the first step's winning LM-head score
    agrees within the fp16 tolerance (ids are compared against the oracle in
    the test above)."""
    uocr = gpu
    m = model(uocr, 3)
    rng = np.random.default_rng(21)
    ids, mask, rows = prompt(rng, 30, 70)
    eng = uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=128, max_gen_tokens=16)
    a_ids, a_sc, _, _ = eng.generate_embeddings(ids, mask, rows, 8, flags=uocr.GEN_IGNORE_EOS)
    b_ids, b_sc, _, _ = eng.generate_embeddings(ids, mask, rows, 8,
                                                flags=uocr.GEN_IGNORE_EOS | uocr.GEN_TOKEN_PREFILL)
    eng.close()
    assert abs(float(a_sc[0]) - float(b_sc[0])) <= 2e-2 + 1e-2 * abs(float(b_sc[0]))


def test_long_prompt_batched_and_token_prefill_agree(gpu):
    """A 1,450-row prompt: 8,700 routed (token, expert) pairs, more than the
    8,192 the bucket build keeps in registers, so its looped path runs; 23
    query tiles of the split flash attention (key chunks of 7 tiles).  The
    MFMA prefill and the per-position prefill agree on the first step's
    winning score within the fp16 tolerance."""
    uocr = gpu
    m = model(uocr, 3)
    rng = np.random.default_rng(31)
    ids, mask, rows = prompt(rng, 50, 1400)
    assert ids.size * 6 > 8192
    eng = uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=1536, max_gen_tokens=8)
    a_ids, a_sc, _, _ = eng.generate_embeddings(ids, mask, rows, 4, flags=uocr.GEN_IGNORE_EOS)
    b_ids, b_sc, _, _ = eng.generate_embeddings(ids, mask, rows, 4,
                                                flags=uocr.GEN_IGNORE_EOS | uocr.GEN_TOKEN_PREFILL)
    eng.close()
    assert a_ids.shape == (4,) and b_ids.shape == (4,)
    assert abs(float(a_sc[0]) - float(b_sc[0])) <= 2e-2 + 1e-2 * abs(float(b_sc[0]))


# vision linear: (qtype, m, k, n, act, split) at the SAM ViT-B global view
# (4096 tokens, 768 wide: qkv 2304 split 768, lin1 3072 + GELU, lin2), the
# CLIP-L view (257 tokens, 1024 wide: qkv split 1024, fc1 4096 + QuickGELU,
# fc2), the projector (2048 -> 1280), the Q4 and fp16 kernels, and ragged
# tiles (m not a multiple of 64, n not a multiple of 128).  Long-K GEMMs on
# grids of fewer than 128 tiles split K (CLIP fc2; 37 K steps in 4 splits of
# 10, 10, 10 and 7 in the 2368-wide case).  n = 100 with k = 192 leaves the
# block's scale region at 300 halves, which the LDS preload copies 2 bytes at
# a time instead of 16.
VISION_CASES = [
    (3, 4096, 768, 2304, 0, 768), (3, 4096, 768, 3072, 2, 0), (3, 4096, 3072, 768, 0, 0),
    (3, 257, 1024, 3072, 0, 1024), (3, 257, 1024, 4096, 1, 0), (3, 257, 4096, 1024, 0, 0),
    (3, 256, 2048, 1280, 0, 0), (4, 257, 1024, 4096, 1, 0), (1, 257, 1024, 4096, 1, 0),
    (1, 4096, 768, 3072, 2, 0), (4, 4096, 768, 2304, 0, 768), (3, 1, 64, 96, 2, 0), (1, 65, 128, 40, 1, 0),
    (4, 100, 192, 96, 2, 32), (3, 100, 2368, 256, 2, 0),
    (3, 37, 192, 100, 0, 0), (4, 37, 192, 100, 1, 0),
]


@pytest.mark.parametrize("qtype,m,k,n,act,split", VISION_CASES)
def test_vision_linear_matches_oracle(gpu, oracle, qtype, m, k, n, act, split):
    """All m rows run on the GPU; the oracle checks the first and last 64 rows
    and 32 random ones (rows are independent)."""
    uocr = gpu
    rng = np.random.default_rng(m + k + n + 10 * act + qtype)
    w, s = weights_for(qtype, rng, n, k)
    x = rand_f16(rng, (m, k))
    bias = rand_f16(rng, n, 0.5)
    dw, ds, db, dx = dev(uocr, w), None if s is None else dev(uocr, s), dev(uocr, bias), dev(uocr, x)
    width = split or n
    outs = [uocr.DeviceBuffer(m * width * 2) for _ in range(3 if split else 1)]
    uocr.op_vision_linear(qtype, dw, ds, db, m, k, n, act, split, dx, *outs)
    uocr.sync()
    got = np.hstack([o.download(np.uint16).reshape(m, width) for o in outs])
    rows = np.unique(np.concatenate([np.arange(min(m, 64)), np.arange(max(0, m - 64), m),
                                     rng.integers(0, m, size=32)]))
    ref = oracle.vision_linear(qtype, w, s, bias.view(np.uint16), rows.size, k, n, act, split,
                               np.ascontiguousarray(x[rows]).view(np.uint16))
    ref = np.hstack(ref) if split else ref
    assert_f16_close(got[rows], ref)


def test_vision_linear_rejects_bad_arguments(gpu):
    uocr = gpu
    buf = uocr.DeviceBuffer(1 << 16)
    with pytest.raises(RuntimeError):
        uocr.op_vision_linear(3, buf, buf, buf, 4, 100, 96, 0, 0, buf, buf)  # k not a multiple of 64
    with pytest.raises(RuntimeError):
        uocr.op_vision_linear(3, buf, buf, None, 4, 128, 96, 0, 0, buf, buf)  # bias is required
    with pytest.raises(RuntimeError):
        uocr.op_vision_linear(3, buf, buf, buf, 4, 128, 96, 3, 0, buf, buf)  # unknown activation
    with pytest.raises(RuntimeError):
        uocr.op_vision_linear(3, buf, buf, buf, 4, 128, 96, 0, 30, buf, buf, buf, buf)  # n != 3 * split
    with pytest.raises(RuntimeError):
        uocr.op_vision_linear(3, buf, buf, buf, 4, 128, 96, 0, 32, buf, buf)  # split needs three outputs


def test_vision_linear_split_k_in_a_graph(gpu, oracle):
    """The CLIP fc2 shape (split K, partials reduced by a second kernel)
    captured into a hipGraph: every replay equals the eager call."""
    uocr = gpu
    rng = np.random.default_rng(5)
    m, k, n = 257, 4096, 1024
    w, s = weights_for(3, rng, n, k)
    x = rand_f16(rng, (m, k))
    bias = rand_f16(rng, n, 0.5)
    dw, ds, db, dx = dev(uocr, w), dev(uocr, s), dev(uocr, bias), dev(uocr, x)
    eager, dy = uocr.DeviceBuffer(m * n * 2), uocr.DeviceBuffer(m * n * 2)
    uocr.op_vision_linear(3, dw, ds, db, m, k, n, 0, 0, dx, eager)
    uocr.sync()
    ref = eager.download(np.uint16)
    with uocr.Capture() as g:
        uocr.op_vision_linear(3, dw, ds, db, m, k, n, 0, 0, dx, dy)
    try:
        for _ in range(3):
            dy.zero()
            g.replay(1)
            uocr.sync()
            assert np.array_equal(dy.download(np.uint16), ref)
    finally:
        g.release()
    rows = np.arange(0, m, 16)
    assert_f16_close(ref.reshape(m, n)[rows], oracle.vision_linear(3, w, s, bias.view(np.uint16), rows.size, k, n, 0,
                                                                   0, np.ascontiguousarray(x[rows]).view(np.uint16)))
