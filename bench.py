"""Benchmark: batch-1 greedy decode of the UnlimitedOCR 12-layer decoder on one MI355X.

Workload: random-init weights of the real decoder
shape (synthetic .uocr image), a prompt of 900 fp16 image-embedding rows
~ N(0,1) plus 32 random text ids (BOS first), then 512 greedy decode steps at
batch 1.  One "step" is one full generate call (prompt processing + 512 decode
steps); `value` is decode tok/s of the mixed-Q4 profile = generated tokens /
decode-loop seconds (src/unlimitedocr_c/perf.py:97-102), weights resident in
HBM before timing starts.  The Q8 and fp16 profiles run the same workload and
are reported beside it.

`roofline` is the dominant kernel of the default Q4 decode, k_decode_run
(one launch of 256 resident workgroups per 8 steps): HIP events around each launch on the
engine stream over one config-5 generation, algorithmic bytes = 8 x the
decode bytes per token.  The Q8 profile decodes through the same run; beside
it, for the per-step graph path (the fp16 default): `graph_path_moe_gate_up`, its dominant kernel k_moe_gate_up at
the decode shape in a hipGraph over expert-slab copies larger than the
Infinity Cache, and `graph_path_kernels`, every per-step kernel's share from
per-launch events (eager launches, dispatch included).  `lm_head_config2` times the Q4
LM-head GEMV + argmax keys (87,912,964 algorithmic bytes
per launch) rotating 6 weight copies (528 MB) so launches stream from HBM
rather than the 256 MB Infinity Cache.
`operators` times BASELINE configs 1, 3 and 4 as single operators through
the C ABI (captured into one hipGraph, HIP events on the operator stream),
weights rotated over copies larger than the Infinity Cache ("cold") and
repeated on one copy ("hot"), with the C oracle's time for the same operator.
`cpu_baseline` is the C oracle's decode step (the restated reference CPU
path) on this host's cores at the same context length, for a bounded number
of tokens.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "unlimitedocr.c_amd"))

import uocr  # noqa: E402

METRIC = "decode tok/s at batch 1 (Q4, Q8, fp16); achieved HBM GB/s vs 8 TB/s peak"
PEAK_HBM = 8.0e12
N_IMAGE, N_TEXT, N_NEW = 900, 32, 512
def tensor_table(model: uocr.SynthModel) -> np.ndarray:
    return uocr.tensor_table(model.view())


def decode_bytes_per_token(model: uocr.SynthModel, prompt_len: int, n_new: int) -> float:
    """Algorithmic HBM bytes per generated token: every weight byte a decode
    step reads (all non-expert tensors, 6 of 64 routed experts per MoE layer,
    one embedding row) plus the KV cache read over the ring attention length
    and the K/V write (61,440 B per token of context)."""
    t = tensor_table(model)
    size = t["payload_size"] + t["scale_size"]
    is_expert = t["family"] == 8
    is_embed = t["family"] == 1
    dense = float(size[~is_expert & ~is_embed].sum())
    experts = float(size[is_expert].sum()) * 6.0 / 64.0
    embed_row = float(size[is_embed].sum()) / 129280.0
    lens = [prompt_len + min(g, 128) for g in range(1, n_new)]
    mean_len = float(np.mean(lens)) if lens else float(prompt_len)
    kv = 61440.0 * (mean_len + 1.0)
    return dense + experts + embed_row + kv


def make_prompt(seed: int = 0):
    rng = np.random.default_rng(seed)
    ids = np.concatenate([[0], np.full(N_IMAGE, 128815), rng.integers(2, 128000, N_TEXT - 1)]).astype(np.int32)
    mask = (ids == 128815).astype(np.uint8)
    rows = rng.standard_normal((N_IMAGE, 1280)).astype(np.float16)
    return ids, mask, rows


def run_profile(qprofile: int, steps: int, warmup: int, log, flags: int = 0) -> dict:
    t0 = time.time()
    model = uocr.synth_model(qprofile, 7)
    ids, mask, rows = make_prompt()
    eng = uocr.Engine.from_memory(model, backend="hip", max_prompt_tokens=1024, max_gen_tokens=N_NEW)
    log(f"profile {qprofile}: model {model.size / 1e9:.2f} GB ready in {time.time() - t0:.1f}s")
    for _ in range(warmup):
        eng.generate_embeddings(ids, mask, rows, N_NEW, flags=uocr.GEN_IGNORE_EOS | flags)
    uocr.sync()
    wall, pre, dec, gen = [], [], [], 0
    for s in range(steps):
        t = time.perf_counter()
        out, _, p_ms, d_ms = eng.generate_embeddings(ids, mask, rows, N_NEW, flags=uocr.GEN_IGNORE_EOS | flags)
        wall.append((time.perf_counter() - t) * 1e3)
        pre.append(p_ms)
        dec.append(d_ms)
        gen += int(out.size)
        log(f"  step {s}: prefill {p_ms:.1f} ms, decode {d_ms:.1f} ms ({out.size / d_ms * 1e3:.1f} tok/s)")
    uocr.sync()
    bpt = decode_bytes_per_token(model, ids.size, N_NEW)
    tok_s = gen / (sum(dec) / 1e3)
    eng.close()
    model.close()
    return {"tok_s": tok_s, "ms_per_step": float(np.mean(wall)), "prefill_ms": float(np.mean(pre)),
            "decode_ms": float(np.mean(dec)), "bytes_per_token": bpt, "hbm_gbs": bpt * tok_s / 1e9,
            "roofline_tok_s": PEAK_HBM / bpt, "frac": bpt * tok_s / PEAK_HBM, "generated": gen}


def _rowbytes(q: str, k: int) -> int:
    """Bytes of one weight row of k inputs: q4_0 / q8_0 payload plus one
    fp16 scale per 64 inputs, or fp16."""
    return {"q4": k // 2 + k // 64 * 2, "q8": k + k // 64 * 2, "f16": 2 * k}[q]


def decode_kernel_bytes(prompt_len: int, n_new: int) -> dict[str, float]:
    """Algorithmic HBM bytes per launch of each config-5 decode kernel, mixed-Q4
    profile (attention projections q8_0, FFN / LM head / embedding q4_0):
    every weight byte the launch needs once, activations in and out once.
    Layer-dependent kernels are averaged over their launches per step."""
    H, I, SI, D0, V = 1280, 896, 1792, 6848, 129280
    act = 2 * H  # one fp16 hidden vector
    att_w = 3 * H * _rowbytes("q8", H)
    # attention length of decode step t (t = 0 .. n_new-2 run the layers): P + min(t + 1, 128)
    lens = [prompt_len + min(t + 1, 128) for t in range(n_new - 1)]
    mean_len = float(np.mean(lens))
    fold = H * 64 * 4  # fp32 router fold, MoE layers (11 of 12)
    return {
        # norm weights + h in, q out, the new K/V rows
        "k_qkv_rope": att_w + 2 * act + act + 2 * act,
        # K and V of every live slot (10 heads x 128 fp16 each) + q in + context out
        "k_attention": 2 * 10 * 128 * 2 * mean_len + 2 * act,
        # O projection + context and residual in, a out, the fold on MoE layers
        "k_attn_out": H * _rowbytes("q8", H) + 3 * act + fold * 11 / 12,
        # routed 6 x (gate, up) rows of 896 + shared merged (gate, up) 1792, a + post norm in, mid out
        "k_moe_gate_up": 6 * 2 * I * _rowbytes("q4", H) + 2 * SI * _rowbytes("q4", H) + 2 * act
                         + 2 * (6 * I + SI),
        # routed 6 x down rows (K = 896) + shared down (K = 1792), mid in, a in, h out
        "k_moe_down": 6 * H * _rowbytes("q4", I) + H * _rowbytes("q4", SI) + 2 * (6 * I + SI) + 2 * act,
        "k_swiglu": 2 * D0 * _rowbytes("q4", H) + 2 * act + 2 * D0,
        "k_gemv": H * _rowbytes("q4", D0) + 2 * D0 + 2 * act,
        "k_lm_keys": V * _rowbytes("q4", H) + 2 * act,
        "k_lm_finalize": _rowbytes("q4", H) + act,
    }


def decode_kernel_roofline(log) -> dict:
    """Per-kernel HBM roofline of the config-5 decode loop (mixed-Q4), timed
    live: one generation of the config-5 workload with the engine's per-launch
    profile events (UOCR_HIP_DECODER_PROFILE_DETAIL=4: eager launches, each
    bracketed by a HIP event pair on the engine's stream, added up per
    kernel).  `achieved` = algorithmic bytes per launch / mean launch time.
    The dominant kernel (largest share of decode time) is the roofline line."""
    os.environ["UOCR_HIP_DECODER_PROFILE_DETAIL"] = "4"
    try:
        model = uocr.synth_model(uocr.QPROFILE_Q4, 7)
        ids, mask, rows = make_prompt()
        with uocr.Engine.from_memory(model, backend="hip", max_prompt_tokens=1024, max_gen_tokens=N_NEW,
                                     profile=True) as eng:
            eng.generate_embeddings(ids, mask, rows, N_NEW, flags=uocr.GEN_IGNORE_EOS)
            eng.profile_reset()
            out, _, _, dec_ms = eng.generate_embeddings(ids, mask, rows, N_NEW, flags=uocr.GEN_IGNORE_EOS)
            ev = eng.profile_events()
        model.close()
    finally:
        del os.environ["UOCR_HIP_DECODER_PROFILE_DETAIL"]
    algo = decode_kernel_bytes(ids.size, N_NEW)
    kern = {k[len("hip.kernel."):]: v for k, v in ev.items() if k.startswith("hip.kernel.")}
    total_ms = sum(v[1] for v in kern.values())
    table = {}
    for name, (calls, ms) in sorted(kern.items(), key=lambda kv: -kv[1][1]):
        us = ms * 1e3 / calls
        gbs = algo[name] / (us * 1e-6) / 1e9
        table[name] = {"launches": calls, "avg_us": round(us, 3), "share": round(ms / total_ms, 4),
                       "algorithmic_bytes": int(algo[name]), "achieved_gbs": round(gbs, 1),
                       "frac": round(gbs / 8000.0, 4)}
    dom = next(iter(table))
    log(f"decode kernels (eager, {out.size} tokens, {dec_ms:.1f} ms, kernel sum {total_ms:.1f} ms): "
        + ", ".join(f"{k} {v['avg_us']:.1f}us x{v['launches']} {v['frac']:.2f}" for k, v in table.items()))
    return {"dominant": dom, "decode_ms": round(dec_ms, 2), "kernel_sum_ms": round(total_ms, 2),
            "timing": "HIP events on the engine stream around each eager launch of one config-5 generation; "
                      "each interval includes the launch's dispatch (about 2 us on this path), so these "
                      "fractions are lower bounds",
            "per_kernel": table}


def gate_up_roofline(log, n_copy: int = 5, per_copy: int = 12, replays: int = 40) -> dict:
    """The dominant config-5 decode kernel, k_moe_gate_up (mixed-Q4: top-6 of
    64 routed experts' gate/up rows 896 x 1280 + the merged shared 1792 x 1280,
    q4_0), at its decode shape through uocr_op_moe_gate_up: n_copy copies of
    the expert slabs (n_copy x 80 MB, more than the 256 MB Infinity Cache),
    each call with fresh N(0,1) router logits (so the selected experts change
    from call to call) and a fresh hidden; the calls are captured into one
    hipGraph and timed with HIP events on the operator stream over `replays`
    replays; mean launch time = elapsed / launches."""
    rng = np.random.default_rng(5)
    E, I, H, SI = 64, 896, 1280, 1792
    keep = []

    def put(a):
        b = uocr.DeviceBuffer.of(np.ascontiguousarray(a))
        keep.append(b)
        return b.ptr

    gw = rng.integers(0, 256, size=(E, I, H // 2), dtype=np.uint8)
    gs = (np.abs(rng.standard_normal((E, I, H // 64))) * 0.02 / 7).astype(np.float16)
    sgw = rng.integers(0, 256, size=(SI, H // 2), dtype=np.uint8)
    sgs = (np.abs(rng.standard_normal((SI, H // 64))) * 0.02 / 7).astype(np.float16)
    mws = []
    for _ in range(n_copy):
        m = uocr.CMoeWeights()
        m.expert_qtype = m.shared_qtype = 4
        m.gate_w, m.gate_s, m.up_w, m.up_s = put(gw), put(gs), put(gw[::-1]), put(gs[::-1])
        m.down_w, m.down_s = m.gate_w, m.gate_s  # not read by the gate/up stage
        m.gu_w_stride, m.gu_s_stride = gw[0].nbytes, gs[0].size
        m.dn_w_stride, m.dn_s_stride = gw[0].nbytes, gs[0].size
        m.sgate_w, m.sgate_s, m.sup_w, m.sup_s = put(sgw), put(sgs), put(sgw[::-1]), put(sgs[::-1])
        m.sdown_w, m.sdown_s = m.sgate_w, m.sgate_s
        mws.append(m)
    n = n_copy * per_copy
    logits = uocr.DeviceBuffer.of(rng.standard_normal((n, E)).astype(np.float32))
    xs = uocr.DeviceBuffer.of(rng.standard_normal((n, H)).astype(np.float16))
    nw = uocr.DeviceBuffer.of(rng.uniform(0.8, 1.2, H).astype(np.float16))
    mid, smid = uocr.DeviceBuffer(n * 6 * I * 2), uocr.DeviceBuffer(n * SI * 2)
    ids, wts = uocr.DeviceBuffer(n * 24), uocr.DeviceBuffer(n * 24)
    calls = [lambda i=i: uocr.op_moe_gate_up(mws[i % n_copy], logits.ptr + i * E * 4, xs.ptr + i * H * 2, nw, 0,
                                             mid.ptr + i * 6 * I * 2, smid.ptr + i * SI * 2, ids.ptr + i * 24,
                                             wts.ptr + i * 24) for i in range(n)]
    ms = _graph_time(log, calls, replays)
    algo = decode_kernel_bytes(N_IMAGE + N_TEXT, N_NEW)["k_moe_gate_up"]
    gbs = algo / (ms / 1e3) / 1e9
    sel = ids.download(np.uint32).reshape(n, 6)
    log(f"k_moe_gate_up (graph, {n} calls x {replays} replays, {n_copy} slab copies): {ms * 1e3:.2f} us/launch, "
        f"{gbs:.0f} GB/s; {len(np.unique(sel))} distinct experts selected")
    traffic = None
    if DECODE_TRAFFIC_FILE.exists():
        traffic = json.loads(DECODE_TRAFFIC_FILE.read_text()).get("k_moe_gate_up", {}).get("hbm_bytes_per_launch")
    return {"kernel": "k_moe_gate_up<Q4, Q4, false> (router top-6 + routed and shared gate/up SwiGLU, config-5 decode "
                      "shape, mixed-Q4)",
            "bound": "hbm", "achieved": round(gbs, 1), "peak": 8000.0, "unit": "GB/s", "frac": round(gbs / 8000.0, 4),
            "traffic": traffic, "avg_launch_us": round(ms * 1e3, 3), "algorithmic_bytes": int(algo),
            "launches": n * replays,
            "timing": f"hipGraph of {n} uocr_op_moe_gate_up calls over {n_copy} expert-slab copies "
                      f"({n_copy * (gw.nbytes + gs.nbytes) * 2 / 1e6:.0f} MB), HIP events around {replays} replays"}


def run_kernel_roofline(log) -> dict:
    """The default Q4 decode: k_decode_run, one launch per 8 decode
    steps (LM head + 12 layers each), timed with an event pair around every
    launch on the engine's stream (UOCR_HIP_RUN_EVENTS=1 with profiling) over
    one config-5 generation.  Algorithmic bytes per launch = 8 x the decode
    bytes per token (decode_bytes_per_token: every weight byte a step reads,
    6 of 64 experts per MoE layer, the KV cache over the attention length)."""
    os.environ["UOCR_HIP_RUN_EVENTS"] = "1"
    try:
        model = uocr.synth_model(uocr.QPROFILE_Q4, 7)
        ids, mask, rows = make_prompt()
        with uocr.Engine.from_memory(model, backend="hip", max_prompt_tokens=1024, max_gen_tokens=N_NEW,
                                     profile=True) as eng:
            eng.generate_embeddings(ids, mask, rows, N_NEW, flags=uocr.GEN_IGNORE_EOS)
            eng.profile_reset()
            out, _, _, dec_ms = eng.generate_embeddings(ids, mask, rows, N_NEW, flags=uocr.GEN_IGNORE_EOS)
            ev = eng.profile_events()
        bpt = decode_bytes_per_token(model, ids.size, N_NEW)
        model.close()
    finally:
        del os.environ["UOCR_HIP_RUN_EVENTS"]
    if "hip.kernel.k_decode_run" not in ev:
        return {}
    launches, ms = ev["hip.kernel.k_decode_run"]
    avg_us = ms * 1e3 / launches
    algo = 8.0 * bpt
    gbs = algo / (avg_us * 1e-6) / 1e9
    log(f"k_decode_run: {launches} launches, {avg_us:.1f} us each ({avg_us / 8:.1f} us/step), {gbs:.0f} GB/s; "
        f"decode loop {dec_ms:.1f} ms for {out.size} tokens")
    traffic = None
    if RUN_TRAFFIC_FILE.exists():
        traffic = json.loads(RUN_TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")
    return {"kernel": "k_decode_run<Q8, Q4, Q4, Q4> (persistent decode run: 8 steps of LM head + 12 layers "
                      "per launch; the default Q4 and Q8 decode)",
            "bound": "hbm", "achieved": round(gbs, 1), "peak": 8000.0, "unit": "GB/s", "frac": round(gbs / 8000.0, 4),
            "traffic": traffic, "avg_launch_us": round(avg_us, 2), "algorithmic_bytes": int(algo),
            "launches": launches,
            "timing": "HIP events around each launch on the engine stream, one config-5 generation"}


RUN_TRAFFIC_FILE = ROOT / "profiles" / "decode_run_q4_traffic.json"
DECODE_TRAFFIC_FILE = ROOT / "profiles" / "decode_q4_config5_traffic.json"
TRAFFIC_FILE = ROOT / "profiles" / "lm_head_q4_traffic.json"


def lm_head_roofline(log, iters: int = 60) -> dict:
    """Q4 LM head 129280x1280 + argmax (config 2), 6 rotating weight copies
    (528 MB > the 256 MB Infinity Cache), HIP events on the operator stream
    around `iters` calls of the dominant kernel alone (uocr_op_lm_head_keys:
    final norm + GEMV + per-block argmax keys); the full operator with the
    token selection (uocr_op_lm_head_argmax, a second one-wavefront launch)
    is timed beside it.  `traffic` comes from the committed rocprofv3 --pmc
    measurement of the same kernel (profiles/lm_head_q4_traffic.json)."""
    rng = np.random.default_rng(1)
    vocab, k = 129280, 1280
    w = rng.integers(0, 256, size=(vocab, k // 2), dtype=np.uint8)
    s = (np.abs(rng.standard_normal((vocab, k // 64))) * 0.02 / 7).astype(np.float16)
    x = rng.standard_normal(k).astype(np.float16)
    copies = [(uocr.DeviceBuffer.of(w), uocr.DeviceBuffer.of(s)) for _ in range(6)]
    dx, ws, keys = uocr.DeviceBuffer.of(x), uocr.workspace(), uocr.DeviceBuffer(16 * 8)
    tok, sc = uocr.DeviceBuffer(4), uocr.DeviceBuffer(4)
    for i in range(6):
        uocr.op_lm_head_keys(4, copies[i][0], copies[i][1], vocab, dx, None, keys)
    uocr.sync()
    with uocr.Timer() as tm:
        for i in range(iters):
            cw, cs = copies[i % 6]
            uocr.op_lm_head_keys(4, cw, cs, vocab, dx, None, keys)
    cold_ms = tm.ms / iters
    with uocr.Timer() as tm:
        for i in range(iters):
            uocr.op_lm_head_keys(4, copies[0][0], copies[0][1], vocab, dx, None, keys)
    hot_ms = tm.ms / iters
    with uocr.Timer() as tm:
        for i in range(iters):
            cw, cs = copies[i % 6]
            uocr.op_lm_head_argmax(4, cw, cs, vocab, dx, None, ws, tok, sc)
    op_ms = tm.ms / iters
    algo = vocab * k // 2 + vocab * (k // 64) * 2 + k * 2 + 4  # + the winner (4 B), as config 2 counts it
    achieved = algo / (cold_ms / 1e3) / 1e9
    log(f"lm head q4 keys: {cold_ms * 1e3:.1f} us rotated ({achieved:.0f} GB/s), {hot_ms * 1e3:.1f} us hot "
        f"({algo / (hot_ms / 1e3) / 1e9:.0f} GB/s); with the selection launch {op_ms * 1e3:.1f} us")
    traffic = None
    if TRAFFIC_FILE.exists():
        traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")
    return {"kernel": "k_lm_keys<Q4> (final norm + Q4 129280x1280 GEMV + per-block argmax keys, config 2)",
            "bound": "hbm", "achieved": round(achieved, 1), "peak": 8000.0, "unit": "GB/s",
            "frac": round(achieved / 8000.0, 4), "traffic": traffic, "avg_launch_us": round(cold_ms * 1e3, 2),
            "hot_cache_achieved": round(algo / (hot_ms / 1e3) / 1e9, 1), "algorithmic_bytes": algo,
            "launches": iters, "with_selection_us": round(op_ms * 1e3, 2)}


def algo_bytes_gemv_q8(rows: int = 6848, k: int = 1280) -> int:
    """Config 1: Q8 payload + fp16 group scales + x + y."""
    return rows * k + rows * (k // 64) * 2 + k * 2 + rows * 2


def algo_bytes_moe_q4() -> int:
    """Config 3 per token: fp16 router + merged shared gate/up/down (1792) +
    6 routed experts (gate/up/down 896), Q4 with scales, + hidden in/out."""
    E, I, H, SI = 64, 896, 1280, 1792
    return E * H * 2 + 3 * (SI * H // 2 + SI * H // 64 * 2) + 6 * 3 * (I * H // 2 + I * H // 64 * 2) + 2 * H * 2


def algo_bytes_attention_q8(context: int) -> int:
    """Config 4: Q8 q/k/v/o (payload + scales) + K and V of `context` slots
    (10 heads x 128 fp16 each) + hidden in/out and the new K/V row."""
    return 4 * (1280 * 1280 + 1280 * 20 * 2) + 5120 * context + 10240


def _q8(rng, rows, k):
    w = rng.integers(-127, 128, size=(rows, k), dtype=np.int8)
    s = (np.abs(rng.standard_normal((rows, k // 64))) * 0.02 / 127).astype(np.float16)
    return w, s


def _q4(rng, rows, k):
    w = rng.integers(0, 256, size=(rows, k // 2), dtype=np.uint8)
    s = (np.abs(rng.standard_normal((rows, k // 64))) * 0.02 / 7).astype(np.float16)
    return w, s


REPLAY_CAP = None  # --op-replays: fewer replays for counter-collection runs


def _graph_time(log, calls, replays: int) -> float:
    """Captures `calls` (a list of zero-argument operator calls) into one
    hipGraph and returns the mean device time per call over `replays`
    replays, HIP events on the operator stream around the replays."""
    if REPLAY_CAP is not None:
        replays = max(1, min(replays, REPLAY_CAP))
    with uocr.Capture() as g:
        for c in calls:
            c()
    try:
        g.replay(1)
        uocr.sync()
        with uocr.Timer() as tm:
            g.replay(replays)
    finally:
        uocr.sync()
        g.release()
    return tm.ms / (replays * len(calls))


def _cpu_time(fn, budget_s: float) -> tuple[float, int]:
    n, t0 = 0, time.perf_counter()
    while n < 2 or time.perf_counter() - t0 < budget_s:
        fn()
        n += 1
    return (time.perf_counter() - t0) / n, n


def _entry(name, algo, cold_ms, hot_ms, cpu_s, cpu_n, cores, note) -> dict:
    cold = algo / (cold_ms / 1e3) / 1e9
    return {"workload": name, "algorithmic_bytes": int(algo), "us_cold": round(cold_ms * 1e3, 3),
            "gbs_cold": round(cold, 1), "frac_cold": round(cold / 8000.0, 4), "us_hot": round(hot_ms * 1e3, 3),
            "gbs_hot": round(algo / (hot_ms / 1e3) / 1e9, 1),
            "cpu": {"us": round(cpu_s * 1e6, 1), "calls": cpu_n, "cores": cores, "kind": "port"},
            "gpu_over_cpu": round(cpu_s / (cold_ms / 1e3), 1), "note": note}


def operator_benchmarks(log, with_cpu: bool = True, cpu_budget_s: float = 2.0) -> dict:
    """BASELINE configs 1, 3 and 4 as single operators through the C ABI.
    Each workload's calls are captured into one hipGraph (no host launch gaps)
    and timed with HIP events on the operator stream.  `cold`: the calls
    rotate over weight copies totalling more than the 256 MB Infinity Cache,
    so weights stream from HBM; `hot`: every call reads the same copy.  The
    C oracle times the same operator on the host cores (bounded sample)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import ctypes as ct

    import oracle

    cores = int(oracle.lib().orc_get_threads())
    out = {}

    # config 1: Q8 GEMV 6848x1280, seed 0, 1000 timed calls
    rng = np.random.default_rng(0)
    w, s = _q8(rng, 6848, 1280)
    x = rng.standard_normal(1280).astype(np.float16)
    n_copy = 60
    copies = [(uocr.DeviceBuffer.of(w), uocr.DeviceBuffer.of(s)) for _ in range(n_copy)]
    dx, dy = uocr.DeviceBuffer.of(x), uocr.DeviceBuffer(6848 * 2)
    cold = _graph_time(log, [lambda c=c: uocr.op_gemv(3, c[0], c[1], 6848, 1280, dx, None, dy) for c in copies],
                       1000 // n_copy + 1)
    hot = _graph_time(log, [lambda: uocr.op_gemv(3, copies[0][0], copies[0][1], 6848, 1280, dx, None, dy)] * n_copy,
                      1000 // n_copy + 1)
    del copies
    xb = x.view(np.uint16)
    cpu_s, cpu_n = _cpu_time(lambda: oracle.gemv(3, w, s, 6848, 1280, xb), cpu_budget_s) if with_cpu else (0.0, 0)
    algo = algo_bytes_gemv_q8()
    out["config1_q8_gemv"] = _entry("Q8_0 GEMV 6848x1280 (k_stream)", algo, cold, hot, cpu_s, cpu_n, cores,
                                    f"{n_copy} weight copies (543 MB) for cold; 1020 calls")
    log(f"config 1: {out['config1_q8_gemv']}")

    # config 3: MoE FFN, 512 consecutive tokens with a fresh hidden each
    rng = np.random.default_rng(3)
    E, I, H, SI = 64, 896, 1280, 1792
    gate = [_q4(rng, I, H) for _ in range(E)]
    up = [_q4(rng, I, H) for _ in range(E)]
    down = [_q4(rng, H, I) for _ in range(E)]
    slab = lambda parts: (np.stack([p[0] for p in parts]), np.stack([p[1] for p in parts]))
    g_, u_, d_ = slab(gate), slab(up), slab(down)
    sg, su, sd = _q4(rng, SI, H), _q4(rng, SI, H), _q4(rng, H, SI)
    router = (rng.standard_normal((E, H)) * 0.03).astype(np.float16)
    nw = rng.uniform(0.8, 1.2, H).astype(np.float16)
    n_tok = 512
    xs = rng.standard_normal((n_tok, H)).astype(np.float16)
    res = rng.standard_normal((n_tok, H)).astype(np.float16)
    keep = []

    def put(a):
        b = uocr.DeviceBuffer.of(a)
        keep.append(b)
        return b.ptr

    mws = []
    for _ in range(5):
        m = uocr.CMoeWeights()
        m.router, m.expert_qtype = put(router), 4
        m.gate_w, m.gate_s, m.up_w, m.up_s = put(g_[0]), put(g_[1]), put(u_[0]), put(u_[1])
        m.down_w, m.down_s = put(d_[0]), put(d_[1])
        m.gu_w_stride, m.gu_s_stride = g_[0][0].nbytes, g_[1][0].size
        m.dn_w_stride, m.dn_s_stride = d_[0][0].nbytes, d_[1][0].size
        m.shared_qtype = 4
        m.sgate_w, m.sgate_s, m.sup_w, m.sup_s = put(sg[0]), put(sg[1]), put(su[0]), put(su[1])
        m.sdown_w, m.sdown_s = put(sd[0]), put(sd[1])
        mws.append(m)
    dxs, dres, dnw = uocr.DeviceBuffer.of(xs), uocr.DeviceBuffer.of(res), uocr.DeviceBuffer.of(nw)
    douts = uocr.DeviceBuffer(n_tok * H * 2)
    wsp, dids, dwts = uocr.workspace(), uocr.DeviceBuffer(24), uocr.DeviceBuffer(24)
    row = lambda buf, t: buf.ptr + t * H * 2

    def moe_call(t, m):
        return lambda: uocr.op_moe_ffn(m, row(dxs, t), dnw, row(dres, t), 0, wsp, row(douts, t), dids, dwts)

    cold = _graph_time(log, [moe_call(t, mws[t % 5]) for t in range(n_tok)], 2)
    hot = _graph_time(log, [moe_call(t, mws[0]) for t in range(n_tok)], 2)
    del keep, mws
    algo = algo_bytes_moe_q4()
    cpu_s, cpu_n = 0.0, 0
    if with_cpu:
        ev = oracle.ExpertView()
        ev.qtype = 4
        ev.gate_w, ev.up_w, ev.down_w = g_[0].ctypes.data, u_[0].ctypes.data, d_[0].ctypes.data
        ev.gate_s, ev.up_s, ev.down_s = g_[1].ctypes.data, u_[1].ctypes.data, d_[1].ctypes.data
        ev.w_stride, ev.s_stride = g_[0][0].nbytes, g_[1][0].size
        xn = oracle.rmsnorm_f16(xs[0].view(np.uint16), nw.view(np.uint16))
        o16, ids6, w6, mg = np.zeros(H, np.uint16), np.zeros(6, np.uint32), np.zeros(6, np.float32), \
            np.zeros(1, np.float32)
        rb = res[0].view(np.uint16)
        a = lambda v: v.ctypes.data
        cpu_s, cpu_n = _cpu_time(lambda: oracle.lib().orc_moe_ffn(
            a(xn), a(rb), a(router), 64, 6, 0, ct.byref(ev), I, 4, a(sg[0]), a(sg[1]), a(su[0]), a(su[1]),
            a(sd[0]), a(sd[1]), SI, a(o16), a(ids6), a(w6), a(mg)), cpu_budget_s)
    out["config3_moe_ffn"] = _entry("MoE FFN Q4: router + 2 shared (1792) + top-6 of 64 routed, per token", algo,
                                    cold, hot, cpu_s, cpu_n, cores,
                                    "512 tokens, fresh hidden each; 5 expert-slab copies (612 MB) for cold")
    log(f"config 3: {out['config3_moe_ffn']}")

    # config 4: attention block (norm, Q8 q/k/v + RoPE + KV write, decode attention, Q8 O + residual)
    for L, n_copy in ((1024, 45), (4096, 20)):
        rng = np.random.default_rng(2)
        cap = L + 128
        W = [_q8(rng, 1280, 1280) for _ in range(4)]
        kc = rng.standard_normal((10, cap, 128)).astype(np.float16)
        vc = rng.standard_normal((10, cap, 128)).astype(np.float16)
        h = rng.standard_normal(1280).astype(np.float16)
        nw = rng.uniform(0.8, 1.2, 1280).astype(np.float16)
        dh, dnw, dout, wsp = uocr.DeviceBuffer.of(h), uocr.DeviceBuffer.of(nw), uocr.DeviceBuffer(2560), \
            uocr.workspace()
        sets = []
        for _ in range(n_copy):
            dw = [(uocr.DeviceBuffer.of(a), uocr.DeviceBuffer.of(b)) for a, b in W]
            sets.append((dw, uocr.DeviceBuffer.of(kc), uocr.DeviceBuffer.of(vc)))

        def att(st):
            dw, dk, dv = st
            return lambda: uocr.op_attention_block(3, dw[0][0], dw[0][1], dw[1][0], dw[1][1], dw[2][0], dw[2][1],
                                                   dw[3][0], dw[3][1], dh, dnw, dk, dv, cap, L, 1, wsp, dout)

        cold = _graph_time(log, [att(st) for st in sets], 4)
        hot = _graph_time(log, [att(sets[0])] * n_copy, 4)
        del sets
        cpu_s, cpu_n = 0.0, 0
        if with_cpu:
            kr = np.ascontiguousarray(kc.transpose(1, 0, 2)).view(np.uint16)
            vr = np.ascontiguousarray(vc.transpose(1, 0, 2)).view(np.uint16)

            def cpu_block():
                n = oracle.rmsnorm_f16(h.view(np.uint16), nw.view(np.uint16))
                q, k, v = (oracle.gemv(3, a, b, 1280, 1280, n) for (a, b) in W[:3])
                q, k = oracle.rope_f16(q, k, L)
                kr[L] = k.reshape(10, 128)
                vr[L] = v.reshape(10, 128)
                ctx = oracle.attention_decode(q, kr, vr, L, 1, L)
                oracle.gemv(3, W[3][0], W[3][1], 1280, 1280, ctx, h.view(np.uint16))

            cpu_s, cpu_n = _cpu_time(cpu_block, cpu_budget_s)
        algo = algo_bytes_attention_q8(L)
        key = f"config4_attention_L{L}"
        out[key] = _entry(f"attention decode layer, Q8 q/k/v/o, context {L}", algo, cold, hot, cpu_s, cpu_n, cores,
                          f"{n_copy} copies of weights + KV for cold")
        log(f"config 4 L={L}: {out[key]}")
    return out


# Vision linears of one encoder block (uocr_metal.m:17111-17180 call sites):
# SAM ViT-B over the 1024 x 1024 global view (64 x 64 = 4096 patches, width
# 768, MLP 3072) and CLIP-L over one view (257 tokens, width 1024, MLP 4096).
VISION_SHAPES = [
    ("sam_qkv", 3, 4096, 768, 2304, 0, 768), ("sam_proj", 3, 4096, 768, 768, 0, 0),
    ("sam_lin1_gelu", 3, 4096, 768, 3072, 2, 0), ("sam_lin2", 3, 4096, 3072, 768, 0, 0),
    ("clip_qkv", 3, 257, 1024, 3072, 0, 1024), ("clip_fc1_quickgelu", 3, 257, 1024, 4096, 1, 0),
    ("clip_fc2", 3, 257, 4096, 1024, 0, 0), ("sam_lin1_gelu_f16", 1, 4096, 768, 3072, 2, 0),
]


def vision_benchmarks(log, with_cpu: bool = True, calls: int = 20, replays: int = 10) -> dict:
    """uocr_op_vision_linear at the SAM / CLIP block shapes: `calls` launches
    captured into one hipGraph, HIP events around `replays` replays.  Bound:
    MFMA (2 m n k flops against the 2.5 PFLOP/s fp16 dense peak).  The C oracle
    computes up to 256 rows of the same linear on the host cores; its time is
    scaled to all m rows."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    cores = int(oracle.lib().orc_get_threads())
    out = {}
    for name, qt, m, k, n, act, split in VISION_SHAPES:
        rng = np.random.default_rng(m + k + n)
        w, s = (_q8(rng, n, k) if qt == 3 else
                ((rng.standard_normal((n, k)) * 0.02).astype(np.float16), None))
        x = rng.standard_normal((m, k)).astype(np.float16)
        bias = (rng.standard_normal(n) * 0.5).astype(np.float16)
        dw, ds = uocr.DeviceBuffer.of(w), None if s is None else uocr.DeviceBuffer.of(s)
        db, dx = uocr.DeviceBuffer.of(bias), uocr.DeviceBuffer.of(x)
        width = split or n
        outs = [uocr.DeviceBuffer(m * width * 2) for _ in range(3 if split else 1)]
        call = lambda: uocr.op_vision_linear(qt, dw, ds, db, m, k, n, act, split, dx, *outs)
        call()  # eager first call: sizes the split-K partials buffer outside the capture
        uocr.sync()
        ms = _graph_time(log, [call] * calls, replays)
        flops = 2.0 * m * n * k
        tf = flops / (ms / 1e3) / 1e12
        entry = {"qtype": {1: "f16", 3: "q8_0"}[qt], "m": m, "k": k, "n": n, "act": act, "split": split,
                 "us": round(ms * 1e3, 2), "tflops": round(tf, 1), "frac_of_2500": round(tf / 2500.0, 4)}
        if with_cpu:
            rows = min(m, 256)
            xs = np.ascontiguousarray(x[:rows]).view(np.uint16)
            cpu_s, cpu_n = _cpu_time(lambda: oracle.vision_linear(qt, w, s, bias.view(np.uint16), rows, k, n, act,
                                                                  split, xs), 1.0)
            entry["cpu"] = {"us_all_rows": round(cpu_s * m / rows * 1e6, 1), "rows_timed": rows, "calls": cpu_n,
                            "cores": cores, "kind": "port"}
        out[name] = entry
        log(f"vision {name}: {entry}")
    return out


def copy_probe(log, nbytes: int = 512 << 20, iters: int = 4) -> None:
    """A plain device-to-device copy of known size: the reference dispatch
    for scaling FETCH_SIZE / WRITE_SIZE counters to bytes."""
    a, b = uocr.DeviceBuffer(nbytes), uocr.DeviceBuffer(nbytes)
    for _ in range(iters):
        uocr.copy(b, a, nbytes)
    uocr.sync()
    log(f"copy probe: {iters} x {nbytes} B device-to-device")


def prefill_flops(prompt_len: int) -> float:
    """GEMM flops of the prompt prefill (2 x active parameters x rows; the LM
    head is not applied to prompt rows) plus causal attention (QK^T and PV over
    the prefix, 10 heads x 128, 12 layers)."""
    H, L = 1280, 12
    attn_w = 4 * H * H
    dense = 3 * H * 6848
    moe = 64 * H + 3 * H * 1792 + 6 * 3 * H * 896
    active = L * attn_w + dense + (L - 1) * moe
    attn = 2 * 2 * 128 * 10 * L * prompt_len * (prompt_len + 1) / 2
    return 2.0 * active * prompt_len + attn


def cpu_baseline(log, budget_s: float = 12.0) -> dict:
    """C oracle decode steps (Q4 profile) at the config-5 context length."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import ctypes as ct

    import oracle

    model = uocr.synth_model(uocr.QPROFILE_Q4, 7)
    orc = oracle.Model(model.ptr, model.size, model, prompt_capacity=1024)
    L = oracle.lib()
    prompt_len = N_IMAGE + N_TEXT
    assert L.orc_session_fill_kv(ct.c_void_p(orc.s), prompt_len + 128, 5) == 1
    assert L.orc_session_reset(ct.c_void_p(orc.s), prompt_len) == 1
    h = (np.random.default_rng(3).standard_normal(1280)).astype(np.float16).view(np.uint16).copy()
    tok, s1, s2 = ct.c_int32(), ct.c_float(), ct.c_float()
    n, t0 = 0, time.perf_counter()
    while n < 3 or time.perf_counter() - t0 < budget_s:
        L.orc_select(ct.c_void_p(orc.s), h.ctypes.data, ct.byref(tok), ct.byref(s1), ct.byref(s2))
        L.orc_forward_token(ct.c_void_p(orc.s), h.ctypes.data, prompt_len + n, None)
        n += 1
    dt = time.perf_counter() - t0
    cores = int(L.orc_get_threads())
    # the same steps on one thread (bounded sample)
    L.orc_set_threads(1)
    n1, t1 = 0, time.perf_counter()
    while n1 < 2 or time.perf_counter() - t1 < budget_s / 3:
        L.orc_select(ct.c_void_p(orc.s), h.ctypes.data, ct.byref(tok), ct.byref(s1), ct.byref(s2))
        L.orc_forward_token(ct.c_void_p(orc.s), h.ctypes.data, prompt_len + n + n1, None)
        n1 += 1
    dt1 = time.perf_counter() - t1
    L.orc_set_threads(cores)
    orc.close()
    model.close()
    log(f"cpu baseline: {n} tokens in {dt:.1f}s on {cores} threads; {n1} tokens in {dt1:.1f}s on 1 thread")
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "single_thread_value": round(n1 / dt1, 3),
            "sample": f"{n} decode steps (LM-head selection + 12 layers) of the mixed-Q4 model at context "
                      f"{prompt_len}-{prompt_len + n}, C oracle with OpenMP over output rows, {dt:.1f} s; "
                      f"then {n1} further steps on 1 thread, {dt1:.1f} s"}


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--profiles", default="q4,q8,fp16", help="comma list of q4,q8,fp16 (q4 is always run)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--roofline-only", action="store_true",
                    help="run only the config-2 LM-head measurement and a copy probe (for rocprofv3 --pmc runs)")
    ap.add_argument("--decode-kernels-only", action="store_true",
                    help="run only the per-kernel roofline of the config-5 decode loop (eager, event-timed)")
    ap.add_argument("--run-only", action="store_true",
                    help="run only the persistent decode kernel's measurement (one config-5 generation) and a copy "
                         "probe (for rocprofv3 runs)")
    ap.add_argument("--gate-up-only", action="store_true",
                    help="run only the dominant-kernel (k_moe_gate_up) graph measurement and a copy probe "
                         "(for rocprofv3 runs)")
    ap.add_argument("--no-ops", action="store_true", help="skip the config 1/3/4 operator measurements")
    ap.add_argument("--ops-only", action="store_true", help="run only the config 1/3/4 operator measurements")
    ap.add_argument("--op-replays", type=int, default=None,
                    help="cap the graph replays of the operator measurements (counter-collection runs)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only the MFMA prefill of the config-5 prompt (Q4 profile, 1 generated token), three times")
    ap.add_argument("--vision-only", action="store_true",
                    help="run only the vision linear (SAM / CLIP block shape) measurements")
    ap.add_argument("--no-vision", action="store_true", help="skip the vision linear measurements")
    ap.add_argument("--no-graph", action="store_true",
                    help="enqueue decode kernels directly instead of replaying hipGraphs (for kernel tracing)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the decode loop runs on a single MI355X (no multi-GPU path)",
              file=sys.stderr)
        sys.exit(2)

    def log(msg: str) -> None:
        print(msg, file=sys.stderr, flush=True)

    if uocr.load_library().uocr_hip_device_count() <= 0:
        log("no HIP device visible")
        sys.exit(1)
    if args.decode_kernels_only:
        print(json.dumps({"decode_kernels": decode_kernel_roofline(log)}), flush=True)
        return
    if args.run_only:
        print(json.dumps({"roofline": run_kernel_roofline(log)}), flush=True)
        copy_probe(log)
        return
    if args.gate_up_only:
        print(json.dumps({"roofline": gate_up_roofline(log)}), flush=True)
        copy_probe(log)
        return
    if args.roofline_only:
        print(json.dumps({"roofline": lm_head_roofline(log)}), flush=True)
        copy_probe(log)
        return
    global REPLAY_CAP
    REPLAY_CAP = args.op_replays
    if args.prefill_only:
        model = uocr.synth_model(uocr.QPROFILE_Q4, 7)
        ids, mask, rows = make_prompt()
        with uocr.Engine.from_memory(model, backend="hip", max_prompt_tokens=1024, max_gen_tokens=8) as eng:
            # the first call runs the prefill eagerly, the second captures it
            # (same prompt length), the third replays the graph
            for _ in range(3):
                _, _, p_ms, _ = eng.generate_embeddings(ids, mask, rows, 1, flags=uocr.GEN_IGNORE_EOS)
        gf = prefill_flops(ids.size)
        print(json.dumps({"prefill": {"ms": round(p_ms, 3), "gflop": round(gf / 1e9, 1),
                                      "tflops": round(gf / (p_ms / 1e3) / 1e12, 1)}}), flush=True)
        return
    if args.vision_only:
        print(json.dumps({"vision": vision_benchmarks(log, not args.no_cpu_baseline)}), flush=True)
        return
    if args.ops_only:
        print(json.dumps({"operators": operator_benchmarks(log, not args.no_cpu_baseline)}), flush=True)
        copy_probe(log)
        return
    names = {"q4": uocr.QPROFILE_Q4, "q8": uocr.QPROFILE_Q8, "fp16": uocr.QPROFILE_FP16}
    wanted = ["q4"] + [p for p in args.profiles.split(",") if p in names and p != "q4"]
    flags = uocr.GEN_NO_GRAPH if args.no_graph else 0
    results = {p: run_profile(names[p], args.steps, args.warmup, log, flags) for p in wanted}
    roof = run_kernel_roofline(log)
    gu = gate_up_roofline(log)
    if not roof:  # no persistent run on this device: the per-step graphs' dominant kernel
        roof = gu
    else:
        roof["graph_path_moe_gate_up"] = gu
    roof["graph_path_kernels"] = decode_kernel_roofline(log)
    lm = lm_head_roofline(log)
    cpu = None if args.no_cpu_baseline else cpu_baseline(log)
    ops = None if args.no_ops else operator_benchmarks(log, not args.no_cpu_baseline)
    vision = None if args.no_vision else vision_benchmarks(log, not args.no_cpu_baseline)
    q4 = results["q4"]
    line = {
        "metric": METRIC,
        "value": round(q4["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(q4["ms_per_step"], 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0/q8_0 weights x fp16 activations -> fp32 accumulate",
        "data": "synthetic: random-init weights (seeded .uocr image), 900 N(0,1) fp16 image rows + 32 random text ids",
        "config": {"workload": "config 5: 12-layer decoder token loop, prompt 900 image rows + 32 text ids, "
                               "512 greedy decode steps, batch 1, mixed-Q4 profile (attention Q8_0)",
                   "prompt_tokens": N_IMAGE + N_TEXT, "decode_steps": N_NEW},
        "roofline": roof,
        "lm_head_config2": lm,
        "cpu_baseline": cpu,
        "prefill": {"ms": round(q4["prefill_ms"], 2), "gflop": round(prefill_flops(N_IMAGE + N_TEXT) / 1e9, 1),
                    "tflops": round(prefill_flops(N_IMAGE + N_TEXT) / (q4["prefill_ms"] / 1e3) / 1e12, 1),
                    "mfma_peak_tflops": 2500.0,
                    "frac": round(prefill_flops(N_IMAGE + N_TEXT) / (q4["prefill_ms"] / 1e3) / 2.5e15, 4),
                    "note": "fp16 MFMA GEMMs + flash attention over the 932-row prompt (Q4 profile); includes the "
                            "host-to-device prompt upload"},
        "operators": ops,
        "vision": vision,
        "decode_hbm": {p: {"tok_s": round(r["tok_s"], 2), "hbm_gbs": round(r["hbm_gbs"], 1),
                           "frac_of_8tbs": round(r["frac"], 4), "roofline_tok_s": round(r["roofline_tok_s"], 1),
                           "bytes_per_token": int(r["bytes_per_token"]), "prefill_ms": round(r["prefill_ms"], 1),
                           "decode_ms": round(r["decode_ms"], 1), "ms_per_step": round(r["ms_per_step"], 1)}
                       for p, r in results.items()},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
