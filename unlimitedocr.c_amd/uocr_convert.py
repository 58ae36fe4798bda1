"""Decoder `.uocr` writer for Hugging Face safetensors checkpoints.

The reference converts a checkpoint with src/unlimitedocr_c/convert.py; this
module covers that path for the tensors the language-model token loop
reads (embedding, LM head, final norm and the 12 decoder layers), so real
weights can run on the HIP engine:

* names -> tensor ids, families, layers, experts and projections follow
  src/unlimitedocr_c/tensor_registry.py:181-240;
* qtypes per profile follow configs/quant-cfg.yaml as the reference runtime
  gates them (mixed-q4: attention Q8_0; embedding, LM head, dense MLP, shared
  and routed experts Q4_0; mixed-q8_0: all of those Q8_0; norms and routers
  stay fp16);
* the bytes come from the library: uocr_quantize_rows (the convert.py
  quantisers, bit-identical) and uocr_image_skeleton_build (header, config,
  tensor directory and the reference's tensor-data layout).

Vision, projector and separator tensors are not part of the token loop; they
are listed in the result as skipped.  Sources are read through the
safetensors header without loading whole files (BF16, F16 or F32 tensors, one
file or an index.json of shards), or given as a mapping of names to arrays.
"""
from __future__ import annotations

import ctypes as ct
import json
import re
import struct
from collections.abc import Mapping
from pathlib import Path

import numpy as np

import uocr

QPROFILES = {"fp16": 1, "mixed-q8_0": 2, "mixed-q4": 3}

# tensor_registry.py: ids, families and projections (include/uocr_format.h)
FAM_TOK_EMBED, FAM_LM_HEAD, FAM_FINAL_NORM, FAM_ATTN, FAM_NORM, FAM_DENSE, FAM_ROUTER, FAM_EXPERT, FAM_SHARED = \
    1, 2, 3, 4, 5, 6, 7, 8, 9
PROJ = {"q_proj": 10, "k_proj": 11, "v_proj": 12, "o_proj": 13, "gate_proj": 20, "up_proj": 21, "down_proj": 22}
LAYER_BASE, LAYER_STRIDE = 10_000, 1_000
_LOCAL = {"input_layernorm": 1, "post_attention_layernorm": 2, "q_proj": 10, "k_proj": 11, "v_proj": 12,
          "o_proj": 13}
_DENSE_LOCAL = {"gate_proj": 30, "up_proj": 31, "down_proj": 32}
_SHARED_LOCAL = {"gate_proj": 50, "up_proj": 51, "down_proj": 52}
_EXPERT_INDEX = {"gate_proj": 0, "up_proj": 1, "down_proj": 2}

_NORM_RE = re.compile(r"^model\.layers\.(\d+)\.(input_layernorm|post_attention_layernorm)\.weight$")
_ATTN_RE = re.compile(r"^model\.layers\.(\d+)\.self_attn\.(q_proj|k_proj|v_proj|o_proj)\.weight$")
_DENSE_RE = re.compile(r"^model\.layers\.0\.mlp\.(gate_proj|up_proj|down_proj)\.weight$")
_ROUTER_RE = re.compile(r"^model\.layers\.(\d+)\.mlp\.gate\.weight$")
_SHARED_RE = re.compile(r"^model\.layers\.(\d+)\.mlp\.shared_experts\.(gate_proj|up_proj|down_proj)\.weight$")
_EXPERT_RE = re.compile(r"^model\.layers\.(\d+)\.mlp\.experts\.(\d+)\.(gate_proj|up_proj|down_proj)\.weight$")


def _layer_id(layer: int, local: int) -> int:
    return LAYER_BASE + layer * LAYER_STRIDE + local


def decoder_entry(name: str) -> tuple[int, int, int, int, int] | None:
    """(tensor id, family, layer, expert, projection) of a decoder tensor
    name (tensor_registry.py:181-240), or None for any other tensor."""
    if name == "model.embed_tokens.weight":
        return 1, FAM_TOK_EMBED, -1, -1, 1
    if name == "lm_head.weight":
        return 2, FAM_LM_HEAD, -1, -1, 1
    if name == "model.norm.weight":
        return 3, FAM_FINAL_NORM, -1, -1, 1
    m = _NORM_RE.match(name)
    if m:
        layer = int(m.group(1))
        return _layer_id(layer, _LOCAL[m.group(2)]), FAM_NORM, layer, -1, 1
    m = _ATTN_RE.match(name)
    if m:
        layer = int(m.group(1))
        return _layer_id(layer, _LOCAL[m.group(2)]), FAM_ATTN, layer, -1, PROJ[m.group(2)]
    m = _DENSE_RE.match(name)
    if m:
        return _layer_id(0, _DENSE_LOCAL[m.group(1)]), FAM_DENSE, 0, -1, PROJ[m.group(1)]
    m = _ROUTER_RE.match(name)
    if m:
        layer = int(m.group(1))
        return _layer_id(layer, 40), FAM_ROUTER, layer, -1, 1
    m = _SHARED_RE.match(name)
    if m:
        layer = int(m.group(1))
        return _layer_id(layer, _SHARED_LOCAL[m.group(2)]), FAM_SHARED, layer, -1, PROJ[m.group(2)]
    m = _EXPERT_RE.match(name)
    if m:
        layer, expert = int(m.group(1)), int(m.group(2))
        local = 100 + expert * 3 + _EXPERT_INDEX[m.group(3)]
        return _layer_id(layer, local), FAM_EXPERT, layer, expert, PROJ[m.group(3)]
    return None


def decoder_tensor_names() -> list[str]:
    """Every decoder tensor name of the checkpoint, in tensor-id order."""
    names = ["model.embed_tokens.weight", "lm_head.weight", "model.norm.weight"]
    for layer in range(12):
        pre = f"model.layers.{layer}."
        names += [pre + "input_layernorm.weight", pre + "post_attention_layernorm.weight"]
        names += [pre + f"self_attn.{p}.weight" for p in ("q_proj", "k_proj", "v_proj", "o_proj")]
        if layer == 0:
            names += [pre + f"mlp.{p}.weight" for p in ("gate_proj", "up_proj", "down_proj")]
            continue
        names.append(pre + "mlp.gate.weight")
        names += [pre + f"mlp.shared_experts.{p}.weight" for p in ("gate_proj", "up_proj", "down_proj")]
        for e in range(64):
            names += [pre + f"mlp.experts.{e}.{p}.weight" for p in ("gate_proj", "up_proj", "down_proj")]
    return names


# ---------------------------------------------------------------------------
# sources
# ---------------------------------------------------------------------------

_DTYPES = {"BF16": (np.uint16, 2), "F16": (np.float16, 2), "F32": (np.float32, 4)}


class SafetensorsSource:
    """Tensors of one safetensors file, or of the shards an index.json
    names, read row ranges at a time from memory maps (8-byte little-endian
    header length, JSON header, then the data block)."""

    def __init__(self, path: str | Path) -> None:
        path = Path(path)
        files: list[Path]
        if path.is_dir():
            index = path / "model.safetensors.index.json"
            if index.exists():
                weight_map = json.loads(index.read_text())["weight_map"]
                files = sorted({path / f for f in weight_map.values()})
            else:
                files = sorted(path.glob("*.safetensors"))
        else:
            files = [path]
        if not files:
            raise FileNotFoundError(f"no safetensors files under {path}")
        self._entries: dict[str, tuple[np.memmap, str, tuple[int, ...], int, int]] = {}
        for f in files:
            with open(f, "rb") as fh:
                (n,) = struct.unpack("<Q", fh.read(8))
                header = json.loads(fh.read(n))
            data = np.memmap(f, dtype=np.uint8, mode="r")
            base = 8 + n
            for name, meta in header.items():
                if name == "__metadata__":
                    continue
                dtype = meta["dtype"]
                if dtype not in _DTYPES:
                    raise ValueError(f"{name}: unsupported dtype {dtype}")
                b, e = meta["data_offsets"]
                shape = tuple(int(d) for d in meta["shape"])
                if e - b != int(np.prod(shape)) * _DTYPES[dtype][1]:
                    raise ValueError(f"{name}: data size does not match shape {shape}")
                self._entries[name] = (data, dtype, shape, base + b, base + e)

    def names(self) -> list[str]:
        return list(self._entries)

    def shape(self, name: str) -> tuple[int, ...]:
        return self._entries[name][2]

    def rows(self, name: str, r0: int, r1: int) -> np.ndarray:
        """Rows [r0, r1) of a rank-2 tensor (rank 1: the whole vector) as
        contiguous fp32; bf16 widens exactly (bits << 16)."""
        data, dtype, shape, b, _ = self._entries[name]
        cols = shape[-1]
        if len(shape) == 1:
            r0, r1 = 0, 1
        npdt, size = _DTYPES[dtype]
        raw = data[b + r0 * cols * size:b + r1 * cols * size].view(npdt).reshape(r1 - r0, cols)
        if dtype == "BF16":
            return (raw.astype(np.uint32) << 16).view(np.float32)
        return np.ascontiguousarray(raw, dtype=np.float32)


class ArraySource:
    """A mapping of names to arrays (any float dtype) as a source."""

    def __init__(self, tensors: Mapping[str, np.ndarray]) -> None:
        self._t = tensors

    def names(self) -> list[str]:
        return list(self._t)

    def shape(self, name: str) -> tuple[int, ...]:
        return tuple(self._t[name].shape)

    def rows(self, name: str, r0: int, r1: int) -> np.ndarray:
        a = self._t[name]
        if a.ndim == 1:
            return np.ascontiguousarray(a.reshape(1, -1), dtype=np.float32)
        return np.ascontiguousarray(a[r0:r1], dtype=np.float32)


# ---------------------------------------------------------------------------
# conversion
# ---------------------------------------------------------------------------

def quantize_rows(qtype: int, values: np.ndarray) -> tuple[np.ndarray, np.ndarray | None]:
    """(payload, scales) of fp32 rows for qtype 1 (f16), 3 (Q8_0) or 4
    (Q4_0), by the library's uocr_quantize_rows."""
    v = np.ascontiguousarray(values, dtype=np.float32)
    rows, cols = v.shape
    if qtype == 1:
        payload, scales = np.empty((rows, cols), np.uint16), None
    else:
        payload = np.empty((rows, cols if qtype == 3 else cols // 2), np.uint8)
        scales = np.empty((rows, cols // 64), np.uint16)
    status = uocr.load_library().uocr_quantize_rows(qtype, v.ctypes.data, rows, cols, payload.ctypes.data,
                                                   None if scales is None else scales.ctypes.data)
    if status != uocr.UOCR_OK:
        raise ValueError(f"quantize_rows(qtype {qtype}, {rows}x{cols}) failed ({status}): non-finite input or bad shape")
    return payload, scales


def convert(source, qprofile: str = "mixed-q4", out_path: str | Path | None = None,
            chunk_rows: int = 4096) -> tuple[uocr.SynthModel, dict]:
    """Converts the decoder tensors of `source` (a SafetensorsSource, a path
    to one, or a mapping of names to arrays) into a .uocr image of
    `qprofile`; writes it to out_path when given.  Returns the image (usable
    with uocr.Engine.from_memory) and a summary."""
    if qprofile not in QPROFILES:
        raise ValueError(f"unknown qprofile {qprofile!r}; expected one of {sorted(QPROFILES)}")
    if isinstance(source, (str, Path)):
        source = SafetensorsSource(source)
    elif isinstance(source, Mapping):
        source = ArraySource(source)
    by_id: dict[int, str] = {}
    skipped = []
    for name in source.names():
        entry = decoder_entry(name)
        if entry is None:
            skipped.append(name)
        else:
            by_id[entry[0]] = name
    image = uocr.SynthModel(QPROFILES[qprofile], None)
    view = image.view()
    table = uocr.tensor_table(view)
    missing = [int(e["id"]) for e in table if int(e["id"]) not in by_id]
    if missing:
        image.close()
        raise ValueError(f"{len(missing)} decoder tensors missing from the source; first tensor id {missing[0]}")
    lib = uocr.load_library()
    hist: dict[int, int] = {}
    for e in table:
        name = by_id[int(e["id"])]
        rank, qtype = int(e["rank"]), int(e["qtype"])
        want = (int(e["lshape"][0]),) if rank == 1 else (int(e["lshape"][0]), int(e["lshape"][1]))
        if source.shape(name) != want:
            image.close()
            raise ValueError(f"{name}: shape {source.shape(name)}, expected {want}")
        rows, cols = (1, want[0]) if rank == 1 else want
        row_bytes = cols * 2 if qtype == 1 else (cols if qtype == 3 else cols // 2)
        groups = cols // 64
        for r0 in range(0, rows, chunk_rows):
            r1 = min(rows, r0 + chunk_rows)
            vals = np.ascontiguousarray(source.rows(name, r0, r1), dtype=np.float32)
            status = lib.uocr_quantize_rows(
                qtype, vals.ctypes.data, r1 - r0, cols, image.ptr + int(e["payload_offset"]) + r0 * row_bytes,
                None if qtype == 1 else image.ptr + int(e["scale_offset"]) + r0 * groups * 2)
            if status != uocr.UOCR_OK:
                image.close()
                raise ValueError(f"{name}: rows {r0}-{r1} could not be converted (non-finite values?)")
        hist[qtype] = hist.get(qtype, 0) + 1
    if out_path is not None:
        with open(out_path, "wb") as f:
            f.write(memoryview(view))
    names = {1: "f16", 3: "q8_0", 4: "q4_0"}
    summary = {"qprofile": qprofile, "tensors": int(table.size), "bytes": int(image.size),
               "qtypes": {names[k]: v for k, v in sorted(hist.items())}, "skipped": sorted(skipped)}
    return image, summary
