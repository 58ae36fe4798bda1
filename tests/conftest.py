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


# quantised formats: the converter's algorithm, restated from convert.py

def convert_q8(values: np.ndarray):
    """convert.py:2058-2063: scale = max|x|/127 (1.0 for an all-zero group), q = clip(rint(x/scale))."""
    rows, cols = values.shape
    g = values.reshape(rows, cols // 64, 64)
    max_abs = np.max(np.abs(g), axis=2)
    scales = np.where(max_abs == 0.0, np.float32(1.0), max_abs / np.float32(127)).astype(np.float32)
    q = np.clip(np.rint(g / scales[:, :, None]), -127, 127).astype(np.int8)
    return q.reshape(rows, cols), scales.astype(np.float16)


def convert_q4(values: np.ndarray):
    """convert.py:2249-2276: signed max / -8 -> fp16 scale, rint/clip to [-8,7], nibble q+8, half-split pack."""
    rows, cols = values.shape
    g = values.reshape(rows, cols // 64, 64)
    idx = np.argmax(np.abs(g), axis=2)
    signed_max = np.take_along_axis(g, idx[:, :, None], axis=2)[:, :, 0]
    s16 = (signed_max / np.float32(-8)).astype(np.float16)
    s32 = s16.astype(np.float32)
    safe = np.where(s32 == 0.0, np.float32(1.0), s32)
    q = np.clip(np.rint(g / safe[:, :, None]), -8, 7).astype(np.int8)
    deq = (q.astype(np.float32) * s32[:, :, None]).reshape(rows, cols)
    biased = (q.astype(np.int16) + 8).astype(np.uint8)
    packed = (biased[:, :, :32] | (biased[:, :, 32:] << 4)).astype(np.uint8)
    return packed.reshape(rows, cols // 2), s16, deq
