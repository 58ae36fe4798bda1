"""The decoder .uocr writer (uocr_convert.py + uocr_quantize_rows +
uocr_image_skeleton_build) against the reference converter's algorithm and
format (src/unlimitedocr_c/convert.py, tensor_registry.py), CPU only.

Pins:
- quantisers: bit-identical to the numpy restatement of convert.py:2058-2063
  (Q8_0) and :2249-2276 (Q4_0) on random rows and on the edge cases numpy
  decides (ties for the largest magnitude, halves under rint, zero groups,
  fp16-subnormal and overflowing scales), plus the reference's own Q4
  round-trip checks (tests/test_convert.py:192-218 in the reference);
- registry: every decoder name maps to the id, family, layer, expert and
  projection of the image directory entry with that id
  (tensor_registry.py:181-240);
- file: an fp16 conversion of the synthetic fp16 image's values reproduces
  its tensor bytes exactly; converted images pass this library's validator
  and the reference's own (src/model/uocr_model_file.c, built into
  oracle/_ref when the reference tree is present); the routed experts of a
  layer are laid out as the reference's contiguous slab (convert.py:863-925).
"""
from __future__ import annotations

import ctypes as ct
import json
import struct
import sys
from pathlib import Path

import numpy as np
import pytest

from conftest import convert_q4, convert_q8

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "unlimitedocr.c_amd"))

REF_MODEL_FILE = ROOT / "oracle" / "_ref" / "libuocr_model_file.so"


@pytest.fixture(scope="module")
def uc(uocr):
    import uocr_convert

    return uocr_convert


def edge_rows() -> np.ndarray:
    rng = np.random.default_rng(11)
    v = (rng.standard_normal((16, 256)) * 0.05).astype(np.float32)
    v[0, :64] = 0.0                        # all-zero group
    v[1, 0], v[1, 5] = 0.5, -0.5           # equal magnitudes: the first sets the sign
    v[2, :64] = np.arange(64, dtype=np.float32) * 0.5 - 8.0  # exact halves under scale 1
    v[2, 0] = -8.0
    v[3, :64] *= 1e-6                      # fp16-subnormal scales
    v[4, 64:128] = rng.uniform(-7e5, 7e5, 64).astype(np.float32)  # Q4 scale overflows fp16
    v[5, 128] = 127.0                      # Q8 scale exactly 1
    v[5, 129:192] = np.arange(63, dtype=np.float32) - 31.5   # halves
    v[6, 192:] = -3.0                      # constant negative group
    return v


@pytest.mark.parametrize("kind", ["random", "edges"])
def test_q8_matches_converter(uc, kind):
    v = edge_rows() if kind == "edges" else (np.random.default_rng(1).standard_normal((64, 1280)) * 0.02).astype(np.float32)
    q, s = uc.quantize_rows(3, v)
    rq, rs = convert_q8(v)
    assert np.array_equal(q.view(np.int8), rq)
    assert np.array_equal(s, rs.view(np.uint16))


@pytest.mark.parametrize("kind", ["random", "edges"])
def test_q4_matches_converter(uc, kind):
    v = edge_rows() if kind == "edges" else (np.random.default_rng(2).standard_normal((64, 1280)) * 0.02).astype(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        rp, rs, _ = convert_q4(v)
    p, s = uc.quantize_rows(4, v)
    assert np.array_equal(p, rp)
    assert np.array_equal(s, rs.view(np.uint16))


def test_f16_matches_numpy_cast(uc):
    v = np.concatenate([edge_rows().ravel(), np.array([65504.0, 65519.0, 65520.0, -7e4, 6e-8, 2.98e-8, 1e-30],
                                                      np.float32)])
    v = v[: v.size // 8 * 8].reshape(-1, 8)
    p, _ = uc.quantize_rows(1, v)
    with np.errstate(over="ignore"):
        assert np.array_equal(p, v.astype(np.float16).view(np.uint16))


def test_q4_pack_roundtrip_reference_checks(uc):
    """The reference's own Q4 checks (tests/test_convert.py:192-218)."""
    rng = np.random.default_rng(7)
    values = rng.standard_normal((4, 128), dtype=np.float32) * 0.05
    values[0, :64] = 0.0
    values[1, 64] = -0.5
    packed, scales = uc.quantize_rows(4, values)
    assert packed.shape == (4, 64) and scales.shape == (4, 2)
    groups = packed.reshape(4, 2, 32)
    q = np.concatenate([(groups & 0x0F).astype(np.int16) - 8, (groups >> 4).astype(np.int16) - 8], axis=2)
    assert q.min() >= -8 and q.max() <= 7
    sc = scales.view(np.float16).astype(np.float32)
    deq = (q.astype(np.float32) * sc[:, :, None]).reshape(4, 128)
    assert np.array_equal(deq[0, :64], np.zeros(64, np.float32))
    assert abs(deq[1, 64] - np.float32(np.float16(-0.5 / -8.0)) * -8.0) < 1e-6
    assert float(np.abs(deq - values).max()) <= float(np.abs(sc).max()) * 0.5 + 1e-6


def test_nonfinite_input_is_rejected(uc):
    v = np.zeros((2, 64), np.float32)
    v[1, 3] = np.inf
    for qt in (1, 3, 4):
        with pytest.raises(ValueError):
            uc.quantize_rows(qt, v)


def test_registry_matches_image_directory(uocr, uc):
    image = uocr.SynthModel(uocr.QPROFILE_Q4, None)
    table = uocr.tensor_table(image.view())
    names = uc.decoder_tensor_names()
    assert len(names) == table.size == 2234
    by_id = {int(e["id"]): e for e in table}
    for n in names:
        tid, fam, layer, expert, proj = uc.decoder_entry(n)
        e = by_id[tid]
        assert (int(e["family"]), int(e["layer"]), int(e["expert"]), int(e["projection"])) == (fam, layer, expert, proj), n
    # known ids (tensor_registry.py: LAYER_BASE 10000, stride 1000, expert base 100, stride 3)
    assert uc.decoder_entry("model.layers.3.self_attn.q_proj.weight")[0] == 13010
    assert uc.decoder_entry("model.layers.1.mlp.experts.0.gate_proj.weight")[0] == 11100
    assert uc.decoder_entry("model.layers.11.mlp.experts.63.down_proj.weight")[0] == 21291
    assert uc.decoder_entry("model.sam_model.blocks.0.attn.qkv.weight") is None
    image.close()


def test_expert_slab_is_contiguous(uocr):
    """convert.py:863-925: per MoE layer, expert payloads back to back in
    (expert, gate/up/down) order, then the scales back to back."""
    for qp in (uocr.QPROFILE_Q4, uocr.QPROFILE_Q8):
        image = uocr.SynthModel(qp, None)
        t = uocr.tensor_table(image.view())
        for layer in range(1, 12):
            ex = t[(t["family"] == 8) & (t["layer"] == layer)]
            ex = ex[np.argsort(ex["id"])]
            assert ex.size == 192
            assert np.all(ex["payload_offset"][1:] == ex["payload_offset"][:-1] + ex["payload_size"][:-1])
            assert np.all(ex["scale_offset"][1:] == ex["scale_offset"][:-1] + ex["scale_size"][:-1])
            assert ex["scale_offset"][0] >= ex["payload_offset"][-1] + ex["payload_size"][-1]
        image.close()


def _ref_validate(image) -> str | None:
    if not REF_MODEL_FILE.exists():
        return None
    lib = ct.CDLL(str(REF_MODEL_FILE))
    lib.uocr_model_file_validate_memory.argtypes = [ct.c_void_p, ct.c_size_t, ct.c_void_p, ct.c_char_p, ct.c_size_t]
    out, err = ct.create_string_buffer(1 << 16), ct.create_string_buffer(512)
    status = lib.uocr_model_file_validate_memory(image.ptr, image.size, out, err, 512)
    return "" if status == 0 else err.value.decode()


@pytest.fixture(scope="module")
def fp16_source(uocr, uc):
    """The synthetic fp16 image's tensors as a name -> fp16 array source."""
    m = uocr.synth_model(uocr.QPROFILE_FP16, 7)
    v = m.view()
    by_id = {uc.decoder_entry(n)[0]: n for n in uc.decoder_tensor_names()}
    src = {}
    for e in uocr.tensor_table(v):
        shape = (int(e["lshape"][0]),) if int(e["rank"]) == 1 else (int(e["lshape"][0]), int(e["lshape"][1]))
        off, size = int(e["payload_offset"]), int(e["payload_size"])
        src[by_id[int(e["id"])]] = v[off:off + size].view(np.float16).reshape(shape)
    yield m, src
    m.close()


def test_fp16_conversion_reproduces_image(uocr, uc, fp16_source):
    m, src = fp16_source
    img, summary = uc.convert(dict(src, **{"model.sam_model.blocks.0.attn.qkv.weight": np.zeros((4, 4))}), "fp16")
    assert summary["qtypes"] == {"f16": 2234}
    assert summary["skipped"] == ["model.sam_model.blocks.0.attn.qkv.weight"]
    a, b = img.view(), m.view()
    ta, tb = uocr.tensor_table(a), uocr.tensor_table(b)
    assert np.array_equal(ta, tb)
    for e in ta:
        off, size = int(e["payload_offset"]), int(e["payload_size"])
        assert np.array_equal(a[off:off + size], b[off:off + size]), int(e["id"])
    assert _ref_validate(img) in (None, "")
    img.close()


def test_mixed_q4_conversion(uocr, uc, fp16_source, tmp_path):
    _, src = fp16_source
    img, summary = uc.convert(src, "mixed-q4", out_path=tmp_path / "m.uocr")
    assert summary["qtypes"] == {"f16": 36, "q8_0": 48, "q4_0": 2150}
    v = img.view()
    t = {int(e["id"]): e for e in uocr.tensor_table(v)}

    def payload(tid, rows=None):
        e = t[tid]
        w = v[int(e["payload_offset"]):int(e["payload_offset"]) + int(e["payload_size"])]
        s = v[int(e["scale_offset"]):int(e["scale_offset"]) + int(e["scale_size"])]
        return w, s

    for name, qt, rows in (("model.embed_tokens.weight", 4, 512), ("model.layers.3.self_attn.q_proj.weight", 3, None),
                           ("model.layers.5.mlp.experts.17.down_proj.weight", 4, None),
                           ("lm_head.weight", 4, 300)):
        vals = src[name].astype(np.float32)[:rows]
        w, s = payload(uc.decoder_entry(name)[0])
        if qt == 3:
            rq, rs = convert_q8(vals)
            assert np.array_equal(w.view(np.int8)[:rq.size], rq.ravel()), name
        else:
            rq, rs, _ = convert_q4(vals)
            assert np.array_equal(w[:rq.size], rq.ravel()), name
        assert np.array_equal(s.view(np.uint16)[:rs.size], rs.view(np.uint16).ravel()), name
    router = uc.decoder_entry("model.layers.4.mlp.gate.weight")[0]
    w, _ = payload(router)
    assert np.array_equal(w.view(np.float16).reshape(64, 1280), src["model.layers.4.mlp.gate.weight"])
    # the file on disk, this library's validator and the reference's
    assert (tmp_path / "m.uocr").stat().st_size == img.size
    eng = uocr.Engine(str(tmp_path / "m.uocr"), backend="cpu-ref")
    eng.close()
    assert _ref_validate(img) in (None, "")
    img.close()


def test_missing_tensor_is_an_error(uc, fp16_source):
    _, src = fp16_source
    partial = dict(src)
    del partial["model.layers.7.mlp.experts.3.up_proj.weight"]
    with pytest.raises(ValueError, match="missing"):
        uc.convert(partial, "mixed-q4")


def _write_safetensors(path: Path, tensors: dict[str, tuple[str, np.ndarray]]) -> None:
    header, blobs, off = {}, [], 0
    for name, (dtype, arr) in tensors.items():
        raw = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dtype, "shape": list(arr.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(h)) + h + b"".join(blobs))


def test_safetensors_source_dtypes_and_shards(uc, tmp_path):
    rng = np.random.default_rng(3)
    a32 = rng.standard_normal((5, 64)).astype(np.float32)
    bf16 = (a32.view(np.uint32) >> 16).astype(np.uint16)  # truncated to bf16
    f16 = rng.standard_normal((3, 64)).astype(np.float16)
    norm = rng.standard_normal(64).astype(np.float32)
    _write_safetensors(tmp_path / "a.safetensors", {"x.bf16": ("BF16", bf16), "x.f32": ("F32", norm)})
    _write_safetensors(tmp_path / "b.safetensors", {"x.f16": ("F16", f16)})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(
        {"weight_map": {"x.bf16": "a.safetensors", "x.f32": "a.safetensors", "x.f16": "b.safetensors"}}))
    s = uc.SafetensorsSource(tmp_path)
    assert sorted(s.names()) == ["x.bf16", "x.f16", "x.f32"]
    assert np.array_equal(s.rows("x.bf16", 1, 4), (bf16[1:4].astype(np.uint32) << 16).view(np.float32))
    assert np.array_equal(s.rows("x.f16", 0, 3), f16.astype(np.float32))
    assert np.array_equal(s.rows("x.f32", 0, 1), norm.reshape(1, -1))
    assert s.shape("x.f32") == (64,)
