"""Shared pytest setup: markers, import paths, built libraries, seeded data."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "unlimitedocr.c_amd"
ORACLE = ROOT / "oracle"
for p in (str(PKG), str(ORACLE)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


def _ensure_built() -> None:
    lib = PKG / "lib" / "libunlimitedocr.so"
    if not lib.exists():
        subprocess.run(["make", "-s", "-C", str(PKG), "-j8"], check=True)
    if not (ORACLE / "liboracle.so").exists():
        subprocess.run(["make", "-s", "-C", str(ORACLE)], check=True)


_ensure_built()


@pytest.fixture(scope="session")
def uocr():
    import uocr as mod
    mod.load_library()
    return mod


@pytest.fixture(scope="session")
def oracle():
    import oracle as mod
    mod.lib()
    return mod


@pytest.fixture(scope="session")
def gpu(uocr):
    if uocr.load_library().uocr_hip_device_count() <= 0:
        pytest.fail("gpu test selected but no HIP device is visible")
    return uocr


@pytest.fixture(scope="session")
def q4_model(uocr):
    return uocr.synth_model(uocr.QPROFILE_Q4, 7)


def rand_f16(rng, shape, scale=1.0) -> np.ndarray:
    return (rng.standard_normal(shape) * scale).astype(np.float16)


def q8_weights(rng, rows, k):
    """int8 uniform [-127,127], fp16 scales |N(0,0.02)|/127 per 64 columns."""
    w = rng.integers(-127, 128, size=(rows, k), dtype=np.int8)
    s = (np.abs(rng.standard_normal((rows, k // 64))) * 0.02 / 127).astype(np.float16)
    return w, s


def q4_weights(rng, rows, k):
    """int4 [-8,7] as half-split nibbles, fp16 scales |N(0,0.02)|/7."""
    w = rng.integers(0, 256, size=(rows, k // 2), dtype=np.uint8)
    s = (np.abs(rng.standard_normal((rows, k // 64))) * 0.02 / 7).astype(np.float16)
    return w, s


def f16_weights(rng, rows, k, scale=0.01):
    return rand_f16(rng, (rows, k), scale), None


def weights_for(qtype, rng, rows, k):
    return {1: f16_weights, 3: q8_weights, 4: q4_weights}[qtype](rng, rows, k)


def dequant(qtype, w, s) -> np.ndarray:
    """Closed form of the storage formats (convert.py:2058-2063, :2266-2274)."""
    if qtype == 1:
        return w.astype(np.float32)
    rows = w.shape[0]
    sc = s.astype(np.float32)
    if qtype == 3:
        k = w.shape[1]
        return (w.astype(np.float32).reshape(rows, k // 64, 64) * sc[:, :, None]).reshape(rows, k)
    k = w.shape[1] * 2
    g = w.reshape(rows, k // 64, 32)
    lo = (g & 15).astype(np.float32) - 8
    hi = (g >> 4).astype(np.float32) - 8
    return (np.concatenate([lo, hi], axis=2) * sc[:, :, None]).reshape(rows, k)
