"""CPU-side checks of the drop-in boundary (no kernel launches).

Covers: every function declared in include/*.h is exported by
libunlimitedocr.so; the public ABI's host behaviour mirrors the reference
engine core (status strings, error text, cpu-ref backend contract of
tests/test_ffi.py:176, request validation of
src/runtime/uocr_request_validation.c, .uocr validation of
src/model/uocr_model_file.c, admission of src/core/uocr_api.c:857-928);
the synthetic model builder writes files the loader accepts.
"""
from __future__ import annotations

import ctypes as ct
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols() -> set[str]:
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        names |= set(re.findall(r"UOCR_API\s+[\w\s\*]+?\b(uocr_\w+)\s*\(", h.read_text()))
    return names


def test_every_declared_symbol_is_exported(uocr):
    lib = uocr.load_library()
    names = declared_symbols()
    assert len(names) >= 35
    for n in sorted(names):
        assert hasattr(lib, n), n
    assert names <= set(uocr.SIGNATURES), names - set(uocr.SIGNATURES)


def test_status_and_category_strings(uocr):
    lib = uocr.load_library()
    assert lib.uocr_abi_version() == (0 << 16) | (1 << 8) | 2
    assert lib.uocr_status_string(0) == b"OK"
    assert lib.uocr_status_string(-4) == b"not implemented"
    assert lib.uocr_status_string(42) == b"unknown status"
    assert lib.uocr_memory_category_name(1) == b"kv-cache"
    assert lib.uocr_memory_category_name(99) == b"unknown"


_PUBLIC_STRUCTS = {"uocr_profile_event": "CProfileEvent", "uocr_memory_report": "CMemoryReport",
                   "uocr_profile_report": "CProfileReport", "uocr_image_view": "CImageView",
                   "uocr_prepared_request": "CPreparedRequest", "uocr_engine_opts": "CEngineOpts"}


def _struct_fields(header: str) -> dict[str, list[str]]:
    """Field names of every public struct of unlimitedocr.h, in order."""
    import re
    text = re.sub(r"/\*.*?\*/", "", Path(header).read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"typedef\s+struct\s+(\w+)\s*\{(.*?)\}\s*\1\s*;", text, flags=re.S):
        names = []
        for decl in m.group(2).split(";"):
            decl = decl.strip()
            if decl:
                names.append(re.findall(r"(\w+)\s*(?:\[[^\]]*\])?\s*$", decl)[0])
        out[m.group(1)] = names
    return out


def _layout(include_dir: str, fields: dict[str, list[str]], tmp: Path) -> dict[str, list[int]]:
    """sizeof and offsetof of every field, compiled by gcc against the
    unlimitedocr.h in include_dir."""
    import subprocess
    lines = ["#include <stddef.h>", "#include <stdio.h>", '#include "unlimitedocr.h"', "int main(void) {"]
    for st, names in fields.items():
        lines.append(f'printf("{st} %zu", sizeof({st}));')
        for n in names:
            lines.append(f'printf(" %zu", offsetof({st}, {n}));')
        lines.append('printf("\\n");')
    lines += ["return 0;", "}"]
    src, exe = tmp / "layout.c", tmp / f"layout_{abs(hash(include_dir))}"
    src.write_text("\n".join(lines))
    subprocess.run(["gcc", "-std=c11", "-I", include_dir, str(src), "-o", str(exe)], check=True)
    res = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    return {ln.split()[0]: [int(v) for v in ln.split()[1:]] for ln in res if ln.strip()}


def test_struct_layouts_match_reference(uocr, tmp_path):
    """Every public struct: sizeof and the offset of every field, compiled
    with offsetof against this build's unlimitedocr.h, equal those compiled
    against the reference's header (where /root/reference is present) and
    those of the ctypes mirror in uocr.py."""
    ours_h = str(ROOT / "include")
    fields = _struct_fields(ours_h + "/unlimitedocr.h")
    assert set(_PUBLIC_STRUCTS) <= set(fields), set(_PUBLIC_STRUCTS) - set(fields)
    ours = _layout(ours_h, fields, tmp_path)
    ref_h = Path("/root/reference/include")
    if (ref_h / "unlimitedocr.h").exists():
        assert _struct_fields(str(ref_h / "unlimitedocr.h")) == fields
        assert _layout(str(ref_h), fields, tmp_path) == ours
    for st, cls in _PUBLIC_STRUCTS.items():
        c = getattr(uocr, cls)
        assert ct.sizeof(c) == ours[st][0], st
        assert [f[0] for f in c._fields_] == fields[st], st
        assert [getattr(c, n).offset for n in fields[st]] == ours[st][1:], st


@pytest.fixture(scope="module")
def cpu_engine(uocr, q4_model):
    eng = uocr.Engine.from_memory(q4_model, backend="cpu-ref", max_prompt_tokens=64, max_gen_tokens=16)
    yield eng
    eng.close()


def test_cpu_ref_validates_but_does_not_generate(uocr, cpu_engine):
    assert cpu_engine.backend == "cpu-ref"
    assert cpu_engine.generate_prepared(np.array([0, 5, 6], np.int32), max_new_tokens=0).size == 0
    with pytest.raises(RuntimeError) as ex:
        cpu_engine.generate_prepared(np.array([0, 5, 6], np.int32), max_new_tokens=2)
    assert ex.value.status == uocr.UOCR_ERROR_NOT_IMPLEMENTED
    assert "max_new_tokens=0" in str(ex.value)


@pytest.mark.parametrize("ids,mask,new,needle", [
    ([5, 6], None, 1, "first token must be BOS"),
    ([0, 129280], None, 1, "out of vocabulary"),
    ([0, 128815], [0, 0], 1, "image_mask is 0"),
    ([0, 7], [0, 1], 1, "expected image token"),
    ([0, 1], [0, 2], 1, "must be 0 or 1"),
    ([0] * 65, None, 1, "engine limit is 64"),
    ([0, 1], None, 17, "engine limit is 16"),
    ([0, 128815, 5, 128815], [0, 1, 0, 1], 1, "contiguous"),
])
def test_request_validation(uocr, cpu_engine, ids, mask, new, needle):
    with pytest.raises(RuntimeError) as ex:
        cpu_engine.generate_prepared(np.array(ids, np.int32), None if mask is None else np.array(mask, np.uint8),
                                     max_new_tokens=new)
    assert ex.value.status == uocr.UOCR_ERROR_INVALID_ARGUMENT
    assert needle in str(ex.value)


def test_reports(uocr, cpu_engine, q4_model):
    rep = cpu_engine.memory_report()
    assert rep.category_live_bytes[0] > 0.9 * q4_model.size  # model views = tensor data
    assert rep.estimated_total_bytes > rep.estimated_model_views_bytes
    prof = cpu_engine.profile_report()
    assert prof.enabled == 0
    lib = uocr.load_library()
    assert lib.uocr_engine_profile_reset(cpu_engine._handle) == 0
    assert lib.uocr_engine_memory_report(None, None) == uocr.UOCR_ERROR_INVALID_ARGUMENT


def test_hip_backend_needs_a_device(uocr, q4_model):
    if uocr.load_library().uocr_hip_device_count() > 0:
        pytest.skip("a HIP device is present")
    with pytest.raises(RuntimeError, match="no HIP device"):
        uocr.Engine.from_memory(q4_model, backend="hip")
    with pytest.raises(RuntimeError, match="Metal backend was not compiled"):
        uocr.Engine.from_memory(q4_model, backend="metal")


def test_memory_budget_admission(uocr, q4_model):
    with pytest.raises(RuntimeError, match="admission rejected"):
        uocr.Engine.from_memory(q4_model, backend="cpu-ref", memory_budget_bytes=1 << 20)


def _open_bytes(uocr, data: bytes, backend="cpu-ref"):
    buf = (ct.c_uint8 * len(data)).from_buffer_copy(data)
    opts = uocr.CEngineOpts(None, backend.encode(), None, 0, 0, 0, 0, 0, 0)
    lib = uocr.load_library()
    h = lib.uocr_engine_open_memory(ct.byref(opts), buf, len(data))
    if h:
        lib.uocr_engine_close(h)
        return None
    return lib.uocr_last_error(None).decode()


@pytest.fixture(scope="module")
def header_bytes(q4_model):
    return bytes(q4_model.view()[:q4_model.size])


def _patched(data: bytes, offset: int, value: bytes) -> bytes:
    b = bytearray(data)
    b[offset:offset + len(value)] = value
    return bytes(b)


def test_model_validation_errors(uocr, header_bytes):
    data = header_bytes
    assert _open_bytes(uocr, data) is None
    assert "bad UOCR magic" in _open_bytes(uocr, _patched(data, 0, b"XOCR"))
    assert "file_size mismatch" in _open_bytes(uocr, data[:-4096])
    assert "config.hidden_size mismatch" in _open_bytes(uocr, _patched(data, 256 + 7 * 4, (1024).to_bytes(4, "little")))
    assert "qprofile" in _open_bytes(uocr, _patched(data, 20, (9).to_bytes(4, "little")))
    # first tensor entry (token embedding, Q4): flip to an unsupported qtype, then an unknown flag
    ent0 = 512 + 16
    assert "unsupported qtype" in _open_bytes(uocr, _patched(data, ent0 + 24, (5).to_bytes(4, "little")))
    assert "unknown flags" in _open_bytes(uocr, _patched(data, ent0 + 28, (0x81).to_bytes(4, "little")))
    # Q4 is not allowed for the attention family (uocr_model_file.c:716-725): retag entry 0 as LAYER_ATTN
    assert "q4_0 is not supported for family" in _open_bytes(uocr, _patched(data, ent0 + 4, (4).to_bytes(4, "little")))
    # ids must ascend
    ent1 = ent0 + 140
    assert "not greater than previous" in _open_bytes(uocr, _patched(data, ent1, (1).to_bytes(4, "little")))


def test_model_file_roundtrip_on_disk(uocr, tmp_path):
    lib = uocr.load_library()
    path = tmp_path / "q4.uocr"
    assert lib.uocr_synth_model_write(str(path).encode(), 3, 3) == 0
    size = path.stat().st_size
    assert size > 1_500_000_000
    eng = uocr.Engine(str(path), backend="cpu-ref")
    assert eng.memory_report().category_live_bytes[0] > 0.99 * size
    eng.close()
    path.unlink()
    with pytest.raises(RuntimeError, match="failed to open model file"):
        uocr.Engine(str(path), backend="cpu-ref")


def test_synth_is_deterministic(uocr):
    a = uocr.synth_model(uocr.QPROFILE_Q8, 11)
    b = uocr.synth_model(uocr.QPROFILE_Q8, 11)
    va, vb = a.view(), b.view()
    assert a.size == b.size
    for off in (0, a.size // 3, a.size // 2, a.size - 65536):
        assert np.array_equal(va[off:off + 65536], vb[off:off + 65536])
    c = uocr.synth_model(uocr.QPROFILE_Q8, 12)
    assert not np.array_equal(va[a.size // 2:a.size // 2 + 4096], c.view()[a.size // 2:a.size // 2 + 4096])
