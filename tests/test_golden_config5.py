"""Consistency of the config-5 oracle fixtures (tests/golden/config5_*.npz,
written by tests/golden/make_config5.py) that the GPU parity test reads.

Recomputing them takes the C oracle minutes per profile, so the CPU suite
checks their invariants instead: shapes and dtypes, ids inside the
vocabulary, each router selection six distinct experts of 64, non-negative
margins, finite fp16 hidden states at the listed checkpoints, and the prompt
the GPU test rebuilds from the seed (its bytes hashed, so a change to
config5_prompt() cannot go unnoticed).
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))

import make_config5  # noqa: E402

PROFILES = ["q4", "q8", "f16"]


@pytest.mark.parametrize("profile", PROFILES)
def test_fixture_invariants(profile):
    fx = np.load(GOLDEN / f"config5_{profile}.npz")
    steps = make_config5.STEPS
    ids, margins, top = fx["ids"], fx["margins"], fx["top"]
    trace, gap = fx["trace"], fx["router_gap"]
    assert ids.shape == (steps,) and ids.dtype == np.int32
    assert ((ids >= 0) & (ids < 129280)).all()
    assert margins.shape == (steps,) and (margins >= 0).all() and np.isfinite(margins).all()
    assert top.shape == (steps,) and np.isfinite(top).all()
    assert trace.shape == (steps - 1, 11, 6) and trace.dtype == np.uint32
    assert (trace < 64).all()
    assert all(len(set(trace[t, l].tolist())) == 6 for t in range(steps - 1) for l in range(11))
    assert gap.shape == (steps, 11)
    assert (gap[:-1] >= 0).all() and np.isfinite(gap[:-1]).all() and np.isinf(gap[-1]).all()
    hs, hidden = fx["hidden_steps"], fx["hidden"]
    assert hidden.shape == (hs.size, 1280) and hidden.dtype == np.uint16
    assert np.isfinite(hidden.view(np.float16).astype(np.float32)).all()
    want = set(range(16, steps, 32)) | {steps - 1}
    assert want <= set(hs.tolist())
    # the first step whose margin is at most 1e-2 is a checkpoint too
    low = np.flatnonzero(margins <= 1e-2)
    if low.size:
        assert int(low[0]) in set(hs.tolist())


def test_prompt_is_stable():
    ids, mask, rows = make_config5.config5_prompt()
    assert ids.shape == (932,) and int(mask.sum()) == 900 and rows.shape == (900, 1280)
    assert ids[0] == 0 and (ids[1:901] == 128815).all() and not mask[0] and not mask[901:].any()
    h = hashlib.sha256(ids.tobytes() + mask.tobytes() + rows.tobytes()).hexdigest()
    assert h == PROMPT_SHA256, h


# sha256 of the prompt (ids, mask, image rows) the fixtures were made from
PROMPT_SHA256 = "65bfb1e58e9b3956aed62925866c6c41ef0c5c19e3a1ae63fe22c1bf3a7c467e"
