"""Writes tests/golden/config5_q{4,8,16}.npz: the C oracle's greedy decode of
BASELINE config 5 (900 N(0,1) fp16 image-embedding rows + 32 text ids, 512
greedy steps) on the synthetic decoder of each quantisation profile
(uocr.synth_model(profile, 7)).

Each fixture holds, per step t < 512: the greedy id, its logit (`top`) and
the oracle's top-2 logit margin; and for the forward pass of step t (which
computes the hidden state step t + 1 selects from, t < 511) the router's
expert ids in layers 1-11 (`trace`), their routing weights (`weights`, raw
softmax probabilities in selection order), each selection's set margin
(`router_gap`, the logit gap between the 6th chosen expert and the best
unchosen one); and the hidden state (fp16 bits, the input of step t's
final norm) at the checkpoint steps `hidden_steps`: every 32nd step from 16, 511, and
the first step whose margin is at most 1e-2.  The prompt is rebuilt from PROMPT_SEED by
config5_prompt(), so the GPU test (tests/test_gpu_engine.py) feeds the HIP
engine the same bytes.

Run from the repository root after `make -C oracle` and
`make -C unlimitedocr.c_amd`:  python tests/golden/make_config5.py [profile ...]
"""
from __future__ import annotations

import ctypes as ct
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
for p in (ROOT / "unlimitedocr.c_amd", ROOT / "oracle"):
    sys.path.insert(0, str(p))

PROMPT_SEED = 5
N_IMAGE, N_TEXT, STEPS = 900, 32, 512
PROFILES = {"q4": 3, "q8": 2, "f16": 1}  # uocr.QPROFILE_*


def config5_prompt():
    """(ids, image_mask, image_rows fp16) of the config-5 prompt."""
    rng = np.random.default_rng(PROMPT_SEED)
    rows = rng.standard_normal((N_IMAGE, 1280)).astype(np.float16)
    text = rng.integers(2, 128000, N_TEXT - 1)
    ids = np.concatenate([[0], np.full(N_IMAGE, 128815), text]).astype(np.int32)
    mask = (ids == 128815).astype(np.uint8)
    return ids, mask, rows


def run(profile: str) -> None:
    import oracle
    import uocr

    lib = oracle.lib()
    lib.orc_session_reset.argtypes = [ct.c_void_p, ct.c_uint32]
    lib.orc_forward_token.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_uint32, ct.c_void_p]
    lib.orc_forward_token_traced.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_uint32, ct.c_void_p, ct.c_void_p,
                                             ct.c_void_p]
    lib.orc_select.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_void_p, ct.c_void_p, ct.c_void_p]
    lib.orc_embed_row.argtypes = [ct.c_uint32, ct.c_void_p, ct.c_void_p, ct.c_uint32, ct.c_uint32, ct.c_int32,
                                  ct.c_void_p]
    m = uocr.synth_model(PROFILES[profile], 7)
    orc = oracle.Model(m.ptr, m.size, m, prompt_capacity=1024)
    ids, mask, rows = config5_prompt()
    P = ids.size
    assert lib.orc_session_reset(orc.s, P) == 1
    h = np.zeros(1280, np.uint16)
    emb = np.zeros(1280, np.uint16)
    t0 = time.time()
    img = 0
    for i in range(P):
        if mask[i]:
            h[:] = rows[img].view(np.uint16)
            img += 1
        else:
            assert orc.embed(int(ids[i]), h) == 1
        assert lib.orc_forward_token(orc.s, oracle.ptr(h), i, None) == 1
    print(f"{profile}: prefill {time.time() - t0:.0f} s", flush=True)
    out_ids = np.zeros(STEPS, np.int32)
    margins = np.zeros(STEPS, np.float32)
    top = np.zeros(STEPS, np.float32)
    trace = np.zeros((STEPS - 1, 11, 6), np.uint32)
    weights = np.zeros((STEPS - 1, 11, 6), np.float32)
    router_gap = np.full((STEPS, 11), np.inf, np.float32)
    checkpoints = set(range(16, STEPS, 32)) | {STEPS - 1}
    saved: dict[int, np.ndarray] = {}
    tok, s1, s2 = ct.c_int32(0), ct.c_float(0.0), ct.c_float(0.0)
    for t in range(STEPS):
        assert lib.orc_select(orc.s, oracle.ptr(h), ct.byref(tok), ct.byref(s1), ct.byref(s2)) == 1
        out_ids[t], margins[t], top[t] = tok.value, s1.value - s2.value, s1.value
        if t in checkpoints or (margins[t] <= 1e-2 and not (margins[:t] <= 1e-2).any()):
            saved[t] = h.copy()
        if t + 1 == STEPS:
            break
        assert orc.embed(tok.value, emb) == 1
        h[:] = emb
        assert lib.orc_forward_token_traced(orc.s, oracle.ptr(h), P + t, oracle.ptr(trace[t]),
                                            oracle.ptr(router_gap[t]), oracle.ptr(weights[t])) == 1
        if t % 64 == 0:
            print(f"{profile}: step {t} ({time.time() - t0:.0f} s)", flush=True)
    np.savez_compressed(Path(__file__).with_name(f"config5_{profile}.npz"), ids=out_ids, margins=margins, top=top,
                        trace=trace, weights=weights, router_gap=router_gap, hidden_steps=np.array(sorted(saved), np.int32),
                        hidden=np.stack([saved[k] for k in sorted(saved)]))
    orc.close()
    print(f"{profile}: done in {time.time() - t0:.0f} s; steps with margin <= 1e-2: "
          f"{int((margins <= 1e-2).sum())}", flush=True)


if __name__ == "__main__":
    for prof in sys.argv[1:] or list(PROFILES):
        run(prof)
