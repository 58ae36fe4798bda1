"""The no-allocation entry point uocr_op_moe_ffn_rows_static against
uocr_op_moe_ffn_rows (the same kernels on a caller workspace): outputs must
be identical, on two calls in a row, the second with fewer rows (the static
scratch keeps the first call's contents, which must not leak into the
second), and more rows than the scratch holds must be rejected."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rand_f16
from test_gpu_ops import _moe_setup, dev

pytestmark = pytest.mark.gpu


def _run_both(uocr, m, rng, P):
    nw = rng.uniform(0.8, 1.2, 1280).astype(np.float16)
    x = rand_f16(rng, (P, 1280))
    res = rand_f16(rng, (P, 1280))
    dx, dnw, dres = dev(uocr, x), dev(uocr, nw), dev(uocr, res)
    ws = uocr.moe_rows_workspace(P)
    ref = uocr.DeviceBuffer(P * 2560)
    got = uocr.DeviceBuffer(P * 2560)
    uocr.op_moe_ffn_rows(m, dx, dnw, dres, P, 0, ws, ref)
    uocr.op_moe_ffn_rows_static(m, dx, dnw, dres, P, 0, got)
    uocr.sync()
    return got.download(np.uint16).reshape(P, 1280), ref.download(np.uint16).reshape(P, 1280)


def test_static_scratch_matches_workspace_entry(gpu):
    uocr = gpu
    rng = np.random.default_rng(2024)
    m, _, keep = _moe_setup(uocr, rng, 4, 4)
    for P in (uocr.STATIC_MAX_ROWS, 9):
        print(f"no-alloc moe_ffn_rows: P={P}", flush=True)
        got, ref = _run_both(uocr, m, rng, P)
        assert np.array_equal(got, ref), f"P={P}: static-scratch output differs from the workspace entry point"
    del keep


def test_static_scratch_rejects_too_many_rows(gpu):
    uocr = gpu
    rng = np.random.default_rng(7)
    m, _, keep = _moe_setup(uocr, rng, 4, 4)
    P = uocr.STATIC_MAX_ROWS + 1
    x = dev(uocr, rand_f16(rng, (P, 1280)))
    out = uocr.DeviceBuffer(P * 2560)
    with pytest.raises(RuntimeError, match="exceed"):
        uocr.op_moe_ffn_rows_static(m, x, None, x, P, 0, out)
    del keep
