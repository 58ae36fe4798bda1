"""End-to-end parity of the HIP decode loop with the CPU oracle.

The engine runs on a synthetic .uocr image at the real decoder shape
(12 layers, 64 experts, vocab 129280); the oracle runs the same prompt on the
same bytes.  Greedy ids must agree while the oracle's top-2 margin exceeds
1e-2 (after the first step whose margin is below that, the two sequences may
legitimately diverge and the comparison stops).
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

_MODELS: dict[int, object] = {}


def model(uocr, qprofile):
    if qprofile not in _MODELS:
        _MODELS.clear()  # keep at most one multi-GB image alive
        _MODELS[qprofile] = uocr.synth_model(qprofile, 7)
    return _MODELS[qprofile]


def compare_ids(got, ref, margins):
    n = 0
    for g, r, m in zip(got, ref, margins):
        if m <= 1e-2:
            break
        assert g == r, f"step {n}: got {g}, oracle {r} (margin {m:.4f})"
        n += 1
    return n


def prompt(rng, n_text, n_image=0):
    ids = np.concatenate([[0], rng.integers(2, 128000, n_text - 1)]).astype(np.int32)
    mask = np.zeros(n_text + n_image, np.uint8)
    if n_image:
        ids = np.concatenate([ids[:1], np.full(n_image, 128815, np.int32), ids[1:]]).astype(np.int32)
        mask[1:1 + n_image] = 1
    rows = (rng.standard_normal((n_image, 1280))).astype(np.float16) if n_image else None
    return ids, mask, rows


@pytest.mark.parametrize("qprofile", [3, 2, 1])
def test_generate_matches_oracle(gpu, oracle, qprofile):
    """Several seeded prompts (text + image rows); every step the oracle
    decides with a margin above 1e-2 must match, and at least one prompt must
    give 3 or more such steps."""
    uocr = gpu
    m = model(uocr, qprofile)
    eng = uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=256, max_gen_tokens=64)
    orc = oracle.Model(m.ptr, m.size, m, prompt_capacity=64)
    best = 0
    for seed in range(4):
        rng = np.random.default_rng(100 * qprofile + seed)
        ids, mask, rows = prompt(rng, 10, 6)
        got, _, _, _ = eng.generate_embeddings(ids, mask, rows, max_new_tokens=10, flags=uocr.GEN_IGNORE_EOS)
        ref, margins = orc.generate(ids, mask, rows.view(np.uint16), max_new=10, ignore_eos=True)
        assert got.shape == (10,)
        best = max(best, compare_ids(got.tolist(), ref.tolist(), margins.tolist()))
        if best >= 3:
            break
    orc.close()
    eng.close()
    assert best >= 3


def test_converted_model_matches_oracle(gpu, oracle):
    """A checkpoint converted by uocr_convert (the fp16 synthetic model's
    values as the source, mixed-q4 output) generates on the HIP engine with
    the greedy ids the oracle computes on the same converted bytes."""
    import sys
    from pathlib import Path

    sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "unlimitedocr.c_amd"))
    import uocr_convert

    uocr = gpu
    m = model(uocr, 1)
    v = m.view()
    by_id = {uocr_convert.decoder_entry(n)[0]: n for n in uocr_convert.decoder_tensor_names()}
    src = {}
    for e in uocr.tensor_table(v):
        shape = (int(e["lshape"][0]),) if int(e["rank"]) == 1 else (int(e["lshape"][0]), int(e["lshape"][1]))
        off, size = int(e["payload_offset"]), int(e["payload_size"])
        src[by_id[int(e["id"])]] = v[off:off + size].view(np.float16).reshape(shape)
    conv, summary = uocr_convert.convert(src, "mixed-q4")
    assert summary["qtypes"]["q4_0"] == 2150
    eng = uocr.Engine.from_memory(conv, backend="hip", max_prompt_tokens=64, max_gen_tokens=16)
    orc = oracle.Model(conv.ptr, conv.size, conv, prompt_capacity=64)
    best = 0
    for seed in range(3):
        rng = np.random.default_rng(700 + seed)
        ids, mask, rows = prompt(rng, 10, 6)
        got, _, _, _ = eng.generate_embeddings(ids, mask, rows, max_new_tokens=8, flags=uocr.GEN_IGNORE_EOS)
        ref, margins = orc.generate(ids, mask, rows.view(np.uint16), max_new=8, ignore_eos=True)
        best = max(best, compare_ids(got.tolist(), ref.tolist(), margins.tolist()))
        if best >= 3:
            break
    orc.close()
    eng.close()
    conv.close()
    assert best >= 3


def test_graph_and_eager_paths_agree(gpu, monkeypatch):
    """The per-step kernels replayed from captured graphs and enqueued
    eagerly give bit-identical ids and scores (the persistent run, which
    computes in another order, is switched off)."""
    monkeypatch.setenv("UOCR_HIP_RUN", "0")
    uocr = gpu
    m = model(uocr, 3)
    rng = np.random.default_rng(5)
    ids, mask, rows = prompt(rng, 12, 4)
    eng = uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=256, max_gen_tokens=40)
    # prefill: eager (first length), eager (no graph), captured (same length
    # again), replayed; then another length eagerly, and the first one again
    a = eng.generate_embeddings(ids, mask, rows, 20, flags=uocr.GEN_IGNORE_EOS)
    b = eng.generate_embeddings(ids, mask, rows, 20, flags=uocr.GEN_IGNORE_EOS | uocr.GEN_NO_GRAPH)
    c = eng.generate_embeddings(ids, mask, rows, 20, flags=uocr.GEN_IGNORE_EOS)
    d = eng.generate_embeddings(ids, mask, rows, 20, flags=uocr.GEN_IGNORE_EOS)
    assert a[0].tolist() == b[0].tolist() == c[0].tolist() == d[0].tolist()
    assert np.array_equal(a[1], b[1]) and np.array_equal(a[1], d[1])
    ids2, mask2, rows2 = prompt(rng, 70, 90)  # 160 rows: three query tiles, split attention
    e1 = eng.generate_embeddings(ids2, mask2, rows2, 8, flags=uocr.GEN_IGNORE_EOS | uocr.GEN_NO_GRAPH)
    e2 = eng.generate_embeddings(ids2, mask2, rows2, 8, flags=uocr.GEN_IGNORE_EOS)
    e3 = eng.generate_embeddings(ids2, mask2, rows2, 8, flags=uocr.GEN_IGNORE_EOS)
    assert e1[0].tolist() == e2[0].tolist() == e3[0].tolist()
    f = eng.generate_embeddings(ids, mask, rows, 20, flags=uocr.GEN_IGNORE_EOS)
    assert f[0].tolist() == a[0].tolist()
    eng.close()


def test_router_fold_matches_router_kernel(gpu, monkeypatch):
    """The decode loop's folded router (logits accumulated by the O kernel,
    selection on the un-normalised logits) against the separate router
    kernel (UOCR_HIP_NO_ROUTER_FOLD=1): while the two id sequences agree,
    every step's winning score agrees within the fp16 tolerance, and the
    first disagreement can only be a near-tie."""
    uocr = gpu
    m = model(uocr, 3)
    rng = np.random.default_rng(31)
    ids, mask, rows = prompt(rng, 20, 8)
    fold = uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=128, max_gen_tokens=40)
    monkeypatch.setenv("UOCR_HIP_NO_ROUTER_FOLD", "1")
    plain = uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=128, max_gen_tokens=40)
    monkeypatch.delenv("UOCR_HIP_NO_ROUTER_FOLD")
    a_ids, a_sc, _, _ = fold.generate_embeddings(ids, mask, rows, 24, flags=uocr.GEN_IGNORE_EOS)
    b_ids, b_sc, _, _ = plain.generate_embeddings(ids, mask, rows, 24, flags=uocr.GEN_IGNORE_EOS)
    fold.close()
    plain.close()
    steps = 0
    for x, y, sx, sy in zip(a_ids.tolist(), b_ids.tolist(), a_sc.tolist(), b_sc.tolist()):
        assert abs(sx - sy) <= 2e-2 + 1e-2 * abs(sy), f"step {steps}: scores {sx} vs {sy}"
        if x != y:
            break
        steps += 1
    assert steps >= 4


def test_ring_window_wrap_matches_oracle(gpu, oracle):
    """More than 128 generated tokens: the KV ring overwrites its oldest slots."""
    uocr = gpu
    m = model(uocr, 3)
    eng = uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=64, max_gen_tokens=160)
    orc = oracle.Model(m.ptr, m.size, m, prompt_capacity=64)
    best = 0
    for seed in range(3):
        rng = np.random.default_rng(9 + seed)
        ids, mask, rows = prompt(rng, 6, 2)
        got = eng.generate_embeddings(ids, mask, rows, 140, flags=uocr.GEN_IGNORE_EOS)[0]
        ref, margins = orc.generate(ids, mask, rows.view(np.uint16), max_new=140, ignore_eos=True)
        n = compare_ids(got.tolist(), ref.tolist(), margins.tolist())
        print(f"ring test seed {seed}: {n} ids compared")
        best = max(best, n)
        if best > 129:
            break
    orc.close()
    eng.close()
    assert best >= 3


def test_text_request_through_public_abi(gpu, oracle):
    """uocr_generate_prepared (the reference's entry point) on a text prompt."""
    uocr = gpu
    m = model(uocr, 3)
    rng = np.random.default_rng(13)
    ids, _, _ = prompt(rng, 9)
    eng = uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=64, max_gen_tokens=16, profile=True)
    assert eng.backend == "hip"
    got = eng.generate_prepared(ids, max_new_tokens=6)
    orc = oracle.Model(m.ptr, m.size, m, prompt_capacity=64)
    ref, margins = orc.generate(ids, max_new=6)
    orc.close()
    assert len(got) == len(ref)
    compare_ids(got.tolist(), ref.tolist(), margins.tolist())
    events = eng.profile_events()
    assert "hip.decode_loop" in events and "hip.prefill" in events
    rep = eng.memory_report()
    assert rep.category_live_bytes[1] > 0  # kv-cache
    with pytest.raises(RuntimeError) as ex:
        eng.generate_prepared(np.array([0, 128815], np.int32), np.array([0, 1], np.uint8), max_new_tokens=2)
    assert getattr(ex.value, "status", None) == uocr.UOCR_ERROR_INVALID_ARGUMENT  # image ids need views
    eng.close()


def test_engine_from_model_file(gpu, tmp_path):
    uocr = gpu
    path = tmp_path / "q4.uocr"
    assert uocr.load_library().uocr_synth_model_write(str(path).encode(), 3, 7) == 0
    eng = uocr.Engine(str(path), backend="hip", max_prompt_tokens=32, max_gen_tokens=8)
    a = eng.generate_prepared(np.array([0, 5, 6, 7], np.int32), max_new_tokens=4)
    eng.close()
    path.unlink()
    m = model(uocr, 3)
    eng2 = uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=32, max_gen_tokens=8)
    b = eng2.generate_prepared(np.array([0, 5, 6, 7], np.int32), max_new_tokens=4)
    eng2.close()
    assert a.tolist() == b.tolist()


def test_separate_engines_on_separate_threads(gpu):
    """include/unlimitedocr.h threading contract: separate engines may run on
    separate threads at the same time.  Two engines generate concurrently
    (ctypes releases the GIL during the call) and give the ids and scores
    each gives alone."""
    import threading

    uocr = gpu
    m = model(uocr, 3)
    rng = np.random.default_rng(61)
    prompts = [prompt(rng, 14, 5), prompt(rng, 9, 3)]
    engines = [uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=64, max_gen_tokens=48) for _ in prompts]
    serial = [e.generate_embeddings(*p, 40, flags=uocr.GEN_IGNORE_EOS) for e, p in zip(engines, prompts)]
    results: list = [None, None]
    errors: list = []

    def run(i):
        try:
            for _ in range(3):
                results[i] = engines[i].generate_embeddings(*prompts[i], 40, flags=uocr.GEN_IGNORE_EOS)
        except Exception as exc:  # surfaced below
            errors.append(exc)

    threads = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    for e in engines:
        e.close()
    assert not errors, errors
    for got, ref in zip(results, serial):
        assert got[0].tolist() == ref[0].tolist()
        assert np.array_equal(got[1], ref[1])


def test_generation_stops_on_eos(gpu, oracle):
    """Sequence rule (uocr_sequence.c:120-166, EOS id 1): generation stops at
    the first EOS, which is returned as the last id.  LM-head row 1 (EOS) is
    overwritten with the row of a token the model picks at some step, so EOS
    ties with it there and wins on the lower id; ids before it are
    unchanged."""
    uocr = gpu
    m = model(uocr, 3)
    rng = np.random.default_rng(23)
    ids, mask, rows = prompt(rng, 10, 4)
    eng = uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=64, max_gen_tokens=16)
    base, _, _, _ = eng.generate_embeddings(ids, mask, rows, 12, flags=uocr.GEN_IGNORE_EOS)
    eng.close()
    base = base.tolist()
    assert 1 not in base
    stop = next(i for i in range(2, len(base)) if base[i] not in base[:i])  # first appearance of a token
    target = base[stop]

    class Image:
        pass

    buf = m.view().copy()
    img = Image()
    img.ptr, img.size, img.keep = buf.ctypes.data, buf.size, buf
    lm = [e for e in uocr.tensor_table(buf) if int(e["id"]) == 2][0]
    row_w, row_s = int(lm["row_size"]), (1280 // 64) * 2
    w0, s0 = int(lm["payload_offset"]), int(lm["scale_offset"])
    buf[w0 + row_w:w0 + 2 * row_w] = buf[w0 + target * row_w:w0 + (target + 1) * row_w]
    buf[s0 + row_s:s0 + 2 * row_s] = buf[s0 + target * row_s:s0 + (target + 1) * row_s]

    eng = uocr.Engine.from_memory(img, backend="hip", max_prompt_tokens=64, max_gen_tokens=16)
    got, _, _, _ = eng.generate_embeddings(ids, mask, rows, 12)
    eng.close()
    orc = oracle.Model(img.ptr, img.size, img, prompt_capacity=64)
    ref, _ = orc.generate(ids, mask, rows.view(np.uint16), max_new=12)
    orc.close()
    assert got.tolist() == base[:stop] + [1]
    assert ref.tolist() == got.tolist()


def test_config5_prompt_matches_oracle(gpu, oracle):
    """BASELINE config 5's prompt at full size: 900 image-embedding rows
    ~ N(0,1) after BOS, then 31 text ids (932 rows through the MFMA
    prefill), then greedy steps; ids must match wherever the oracle's margin
    exceeds 1e-2 (the oracle runs the prompt position by position)."""
    uocr = gpu
    m = model(uocr, 3)
    rng = np.random.default_rng(0)
    ids = np.concatenate([[0], np.full(900, 128815), rng.integers(2, 128000, 31)]).astype(np.int32)
    mask = (ids == 128815).astype(np.uint8)
    rows = rng.standard_normal((900, 1280)).astype(np.float16)
    eng = uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=1024, max_gen_tokens=16)
    got, _, _, _ = eng.generate_embeddings(ids, mask, rows, 6, flags=uocr.GEN_IGNORE_EOS)
    eng.close()
    orc = oracle.Model(m.ptr, m.size, m, prompt_capacity=1024)
    ref, margins = orc.generate(ids, mask, rows.view(np.uint16), max_new=6, ignore_eos=True)
    orc.close()
    assert got.shape == (6,)
    assert margins[0] > 1e-2, "seed gives a first step without a clear winner"
    assert compare_ids(got.tolist(), ref.tolist(), margins.tolist()) >= 1


@pytest.mark.parametrize("where,run", [("prefill", "0"), ("decode", "0"), ("decode", "1")])
def test_hot_path_allocation_fails_the_request(gpu, monkeypatch, where, run):
    """The hot-path allocation guard (uocr_metal.m:8447-8486 semantics): a
    device allocation inside the prompt prefill or the decode loop fails the
    request with UOCR_ERROR_INTERNAL naming the region.  The allocation is
    forced by the UOCR_HIP_FAULT_ALLOC test hook; without it the same request
    succeeds (graph path, and the persistent run with UOCR_HIP_RUN=1)."""
    uocr = gpu
    m = model(uocr, 3)
    rng = np.random.default_rng(11)
    ids, mask, rows = prompt(rng, 8, 4)
    monkeypatch.setenv("UOCR_HIP_RUN", run)
    with uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=64, max_gen_tokens=16) as eng:
        got, _, _, _ = eng.generate_embeddings(ids, mask, rows, max_new_tokens=4, flags=uocr.GEN_IGNORE_EOS)
        assert got.shape == (4,)
        assert eng.decode_path() == (1 if run == "1" else 0)
    monkeypatch.setenv("UOCR_HIP_FAULT_ALLOC", where)
    with uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=64, max_gen_tokens=16) as eng:
        with pytest.raises(RuntimeError) as ex:
            eng.generate_embeddings(ids, mask, rows, max_new_tokens=4, flags=uocr.GEN_IGNORE_EOS)
        assert ex.value.status == uocr.UOCR_ERROR_INTERNAL
        assert "allocated device memory" in str(ex.value)
        assert ("prefill" if where == "prefill" else "decode loop") in str(ex.value)


@pytest.mark.parametrize("run", ["0", "1"])
def test_trace_of_a_shorter_generation(gpu, monkeypatch, run):
    """The decode trace of a generation shorter than the traced step count:
    the steps it reaches hold its expert ids and weights (6 distinct ids per
    layer, weights in (0, 1] and summing to at most 1 per layer), every later
    step reads 0xffffffff ids and NaN weights, also after a longer traced
    generation filled them."""
    uocr = gpu
    m = model(uocr, 3)
    rng = np.random.default_rng(41)
    ids, mask, rows = prompt(rng, 8, 4)
    monkeypatch.setenv("UOCR_HIP_RUN", run)
    with uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=64, max_gen_tokens=16) as eng:
        eng.trace_enable(12)
        eng.generate_embeddings(ids, mask, rows, max_new_tokens=13, flags=uocr.GEN_IGNORE_EOS)
        long_ids, _ = eng.trace_read()
        assert (long_ids != 0xFFFFFFFF).all()
        eng.generate_embeddings(ids, mask, rows, max_new_tokens=5, flags=uocr.GEN_IGNORE_EOS)
        assert eng.decode_path() == (1 if run == "1" else 0)
        sel, _ = eng.trace_read()
        w = eng.trace_read_weights()
    assert (sel[:4] < 64).all() and (sel[4:] == 0xFFFFFFFF).all()
    assert np.isnan(w[4:]).all() and not np.isnan(w[:4]).any()
    assert all(len(set(sel[t, l].tolist())) == 6 for t in range(4) for l in range(11))
    assert (w[:4] > 0).all() and (w[:4] <= 1).all() and (w[:4].sum(axis=2) <= 1 + 1e-5).all()
    assert (sel[:4] == long_ids[:4]).all()


def test_forced_run_fails_where_unsupported(gpu, monkeypatch):
    """UOCR_HIP_RUN=1 forces the persistent run: an fp16 model, which has no
    run kernel, fails the engine's creation with a message naming the run
    instead of decoding on the per-step kernels."""
    uocr = gpu
    m = model(uocr, 1)
    monkeypatch.setenv("UOCR_HIP_RUN", "1")
    with pytest.raises(RuntimeError) as ex:
        uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=64, max_gen_tokens=16)
    assert "persistent decode run" in str(ex.value)


def test_run_timeout_serves_the_request_again(gpu, monkeypatch):
    """A persistent run that gives up waiting (forced from the host with a
    zero wait limit, UOCR_HIP_RUN_LIMIT_US=0: every workgroup leaves the
    kernel normally once one of them raises the abort word) is served again
    on the per-step kernels: decode_path() reports 2 and the ids equal the
    per-step path's."""
    uocr = gpu
    m = model(uocr, 3)
    rng = np.random.default_rng(51)
    ids, mask, rows = prompt(rng, 8, 4)
    monkeypatch.setenv("UOCR_HIP_RUN", "0")
    with uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=64, max_gen_tokens=16) as eng:
        ref, _, _, _ = eng.generate_embeddings(ids, mask, rows, max_new_tokens=12, flags=uocr.GEN_IGNORE_EOS)
    monkeypatch.setenv("UOCR_HIP_RUN", "1")
    monkeypatch.setenv("UOCR_HIP_RUN_LIMIT_US", "0")
    with uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=64, max_gen_tokens=16) as eng:
        got, _, _, _ = eng.generate_embeddings(ids, mask, rows, max_new_tokens=12, flags=uocr.GEN_IGNORE_EOS)
        assert eng.decode_path() == 2
    assert got.tolist() == ref.tolist()


def test_per_op_decode_profile_events(gpu, monkeypatch):
    """Profiling on and UOCR_HIP_DECODER_PROFILE_DETAIL=3: the decode loop
    runs eagerly with an event pair around each launch and reports
    hip.decode.* roles (uocr_metal.m:14338-14496 names) with one call per
    launch, the same greedy ids as the graph path, and per-launch times that
    sum to no more than the decode loop's wall time."""
    uocr = gpu
    m = model(uocr, 3)
    rng = np.random.default_rng(21)
    ids, mask, rows = prompt(rng, 8, 4)
    N = 4
    with uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=64, max_gen_tokens=16) as eng:
        ref, _, _, _ = eng.generate_embeddings(ids, mask, rows, max_new_tokens=N, flags=uocr.GEN_IGNORE_EOS)
    monkeypatch.setenv("UOCR_HIP_DECODER_PROFILE_DETAIL", "3")
    with uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=64, max_gen_tokens=16, profile=True) as eng:
        got, _, _, dms = eng.generate_embeddings(ids, mask, rows, max_new_tokens=N, flags=uocr.GEN_IGNORE_EOS)
        ev = eng.profile_events()
    assert got.tolist() == ref.tolist()
    steps = N - 1  # the last step runs the LM head only
    assert ev["hip.decode.attention"][0] == 12 * steps
    assert ev["hip.decode.attention_projections"][0] == 2 * 12 * steps
    assert ev["hip.decode.dense_mlp"][0] == 2 * steps
    assert ev["hip.decode.moe_routed_experts"][0] == 2 * 11 * steps
    assert ev["hip.decode.layer"][0] == 12 * steps
    assert ev["hip.decode.lm_head"][0] >= N
    per_op = sum(v[1] for k, v in ev.items() if k.startswith("hip.decode.") and k != "hip.decode.layer")
    assert 0.0 < per_op <= dms


# Router set margins (logit units) at or below which the engine's expert set
# may differ from the oracle's: the parity contract's 1e-2 (expert ids exact
# wherever the margin exceeds it).
ROUTER_TIE = 1e-2
# Routing weights (raw softmax probabilities) of matching selections: the
# reference's router-weight threshold (parity_thresholds.py:66-70).
ROUTER_WEIGHT_ATOL = 5e-5
# End to end (engine against the oracle's fixture) the router input itself
# differs by fp16 rounding-order effects; measured on config 5: at most
# 1.5e-3 absolute, 0.94% relative.
ROUTER_WEIGHT_RTOL_E2E = 1.5e-2
# Steps after a routing difference whose ids are not compared: the other
# expert's output stays in that step's KV row (a mismatch at margin 0.014
# was seen four steps after such a difference).
FLIP_WINDOW = 8


@pytest.mark.parametrize("profile,run", [("q4", "0"), ("q4", "1"), ("q8", "0"), ("q8", "1"), ("f16", "0")])
def test_config5_full_decode_matches_oracle(gpu, monkeypatch, profile, run):
    """BASELINE config 5 end to end: the 932-row prompt of
    tests/golden/make_config5.py and 512 greedy steps against the C oracle's
    fixture for the same synthetic model (seed 7).

    Teacher-forced (the engine embeds the oracle's token after each step, so
    every step is a function of the oracle's prefix):
    - router: in each of the 511 forward passes, the first layer whose expert
      set differs from the oracle's must be one where the oracle's set margin
      is at most ROUTER_TIE (a near-tie; the later layers of that pass see a
      different hidden state); in every layer before it (outside the window
      after a difference) each selected expert's routing weight is within
      ROUTER_WEIGHT_ATOL + ROUTER_WEIGHT_RTOL_E2E * w of the oracle's;
    - router arithmetic: on the engine's own traced router input (every third
      forward pass), the reference router (fp16 rmsnorm, fp32 logits, raw
      softmax) gives the engine's expert set unless its set margin is at most
      ROUTER_TIE, and each weight within ROUTER_WEIGHT_ATOL (5e-5);
    - ids and logits: at every step whose oracle margin exceeds 1e-2 and
      whose last FLIP_WINDOW forward passes took the oracle's experts, the
      engine's argmax equals the oracle's id and its logit is within
      2e-2 + 1e-2 |logit| of the oracle's; at least 128 steps compared;
    - hidden state (the final norm's input) at the fixture checkpoints with
      no routing difference in the window before them:
      |got - ref| <= 2e-2 + 1e-2 |ref|.
    Free-running (the production path, no trace or forcing): ids equal the
    oracle's up to the first step with a margin of at most 1e-2 or after a
    router near-tie.
    run "1" takes the persistent decode (UOCR_HIP_RUN=1) where
    the profile has one; "0" the per-step kernel path."""
    import sys
    from pathlib import Path

    golden = Path(__file__).resolve().parent / "golden"
    sys.path.insert(0, str(golden))
    import make_config5
    import oracle as oracle_mod

    uocr = gpu
    fx = np.load(golden / f"config5_{profile}.npz")
    ref, margins, top, trace, gap = fx["ids"], fx["margins"], fx["top"], fx["trace"], fx["router_gap"]
    steps = ref.size
    monkeypatch.setenv("UOCR_HIP_RUN", run)
    m = model(uocr, make_config5.PROFILES[profile])
    ids, mask, rows = make_config5.config5_prompt()
    with uocr.Engine.from_memory(m, backend="hip", max_prompt_tokens=1024, max_gen_tokens=steps) as eng:
        free, _, _, _ = eng.generate_embeddings(ids, mask, rows, max_new_tokens=steps, flags=uocr.GEN_IGNORE_EOS)
        # step t selects from the hidden state of forward pass t - 1
        tie = np.concatenate([[False], gap[:-1].min(axis=1) <= ROUTER_TIE])
        amb = (margins <= 1e-2) | np.maximum.accumulate(tie)
        first_amb = int(np.argmax(amb)) if amb.any() else steps
        assert free[:first_amb].tolist() == ref[:first_amb].tolist(), "free-running ids before the first ambiguous step"

        eng.trace_force(ref)
        eng.trace_enable(steps - 1)
        got, score, _, _ = eng.generate_embeddings(ids, mask, rows, max_new_tokens=steps, flags=uocr.GEN_IGNORE_EOS)
        sel, hidden = eng.trace_read()
        wts = eng.trace_read_weights()
        assert eng.decode_path() == (1 if run == "1" else 0), "decode path taken"
        assert got.shape == (steps,)
        flipped = np.zeros(steps + FLIP_WINDOW, bool)
        wref = fx["weights"]
        werr = []
        for t in range(steps - 1):
            diff = [layer for layer in range(11) if sorted(sel[t, layer]) != sorted(trace[t, layer])]
            if diff:
                assert gap[t, diff[0]] <= ROUTER_TIE, \
                    f"forward {t} layer {diff[0] + 1}: experts {sorted(sel[t, diff[0]])} vs oracle " \
                    f"{sorted(trace[t, diff[0]])} at set margin {gap[t, diff[0]]:.4f}"
            if not flipped[t]:
                for layer in range(diff[0] if diff else 11):
                    want = dict(zip(trace[t, layer].tolist(), wref[t, layer].tolist()))
                    for e, w in zip(sel[t, layer].tolist(), wts[t, layer].tolist()):
                        werr.append((abs(w - want[e]), want[e], t, layer))
            if diff:
                flipped[t + 1:t + 1 + FLIP_WINDOW] = True
        # routing weights against the fixture: the engine's hidden state
        # differs from the oracle's by fp16 rounding-order effects (MFMA
        # prefill, split attention), which move the logits by ~1e-3
        err = np.array([x[0] for x in werr])
        ref_w = np.array([x[1] for x in werr])
        assert err.size >= 6 * 11 * 128, f"only {err.size} routing weights compared"
        bad = np.flatnonzero(err > ROUTER_WEIGHT_ATOL + ROUTER_WEIGHT_RTOL_E2E * ref_w)
        assert bad.size == 0, f"routing weight {werr[bad[0]]} beyond the end-to-end bound"
        # the router itself, on the engine's own router input: the reference
        # arithmetic (rmsnorm rounded to fp16, fp32 logits, raw softmax) on the
        # traced a gives the engine's ids (set margin above ROUTER_TIE) and
        # its weights within ROUTER_WEIGHT_ATOL
        inputs = eng.trace_read_router_inputs()
        image = m.view()
        by_id = {int(e["id"]): e for e in uocr.tensor_table(image)}
        rw = [uocr.f16_tensor(image, by_id[10040 + 1000 * l], 64, 1280).view(np.uint16).copy() for l in range(1, 12)]
        pn = [uocr.f16_tensor(image, by_id[10002 + 1000 * l], 1, 1280).view(np.uint16)[0].copy() for l in range(1, 12)]
        worst, n_w = 0.0, 0
        for t in range(0, steps - 1, 3):
            for layer in range(11):
                n2 = oracle_mod.rmsnorm_f16(inputs[t, layer], pn[layer])
                ids_o, w_o, probs, _ = oracle_mod.router_topk(n2, rw[layer])
                order = np.sort(probs)[::-1]
                set_margin = float(np.log(order[5]) - np.log(order[6]))
                if sorted(ids_o.tolist()) != sorted(sel[t, layer].tolist()):
                    assert set_margin <= ROUTER_TIE, f"forward {t} layer {layer + 1}: router on the engine's input"
                    continue
                want = dict(zip(ids_o.tolist(), w_o.tolist()))
                for e, w in zip(sel[t, layer].tolist(), wts[t, layer].tolist()):
                    d = abs(w - want[e])
                    assert d <= ROUTER_WEIGHT_ATOL, \
                        f"forward {t} layer {layer + 1} expert {e}: weight {w:.7f} vs reference router {want[e]:.7f}"
                    worst, n_w = max(worst, d), n_w + 1
        assert n_w >= 6 * 11 * 150
        print(f"routing weights: {err.size} against the fixture (max |diff| {err.max():.2e}, "
              f"max rel {(err / ref_w).max():.2e}); {n_w} against the reference router on the engine's input "
              f"(max |diff| {worst:.2e})")
        comparable = (margins > 1e-2) & ~flipped[:steps]
        bad = np.flatnonzero(comparable & (got != ref))
        assert bad.size == 0, f"forced steps {bad[:8].tolist()}: got {got[bad[:8]].tolist()}, oracle {ref[bad[:8]].tolist()}"
        np.testing.assert_allclose(score[comparable], top[comparable], atol=2e-2, rtol=1e-2)
        assert int(comparable.sum()) >= 128, f"only {int(comparable.sum())} steps compared"
        checked = 0
        for k, href in zip(fx["hidden_steps"], fx["hidden"]):
            k = int(k)
            if flipped[k]:
                continue
            if k + 1 < steps:
                eng.generate_embeddings(ids, mask, rows, max_new_tokens=k + 1, flags=uocr.GEN_IGNORE_EOS)
                _, h = eng.trace_read()
            else:
                h = hidden
            want = href.view(np.float16).astype(np.float32)
            np.testing.assert_allclose(h.astype(np.float32), want, atol=2e-2, rtol=1e-2,
                                       err_msg=f"hidden state at step {k}")
            checked += 1
        assert checked >= 4
