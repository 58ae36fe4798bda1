"""Turn the reference's tiny golden tensors into a JSON data fixture.

Source: tests/fixtures/cpu_ref_tiny_golden.h of the reference (generated there
by tools/uocr-dump-cpu-ref-tiny from NumPy).  Only the numbers (the `#define`
scalars and `static const` arrays) are carried over, as data; the output is
tests/golden/cpu_ref_tiny_golden.json.  Run in a container that has the
reference tree:  python tests/golden/extract_cpu_ref_tiny.py [REF_ROOT]
"""
import json
import re
import sys
from pathlib import Path

ref_root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
src = (ref_root / "tests/fixtures/cpu_ref_tiny_golden.h").read_text()

out = {}
for name, value in re.findall(r"#define (UOCR_TINY_\w+) ([-+0-9.eE]+)[uf]?\n", src):
    out[name] = float(value) if any(ch in value for ch in ".eE") else int(value)
for kind, name, body in re.findall(r"static const (float|uint32_t) (UOCR_TINY_\w+)\[\w+\] = \{(.*?)\};", src, re.S):
    items = [tok.strip().rstrip("uf") for tok in body.split(",") if tok.strip()]
    out[name] = [float(t) for t in items] if kind == "float" else [int(t) for t in items]

dest = Path(__file__).with_name("cpu_ref_tiny_golden.json")
dest.write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
print(f"wrote {dest} ({len(out)} entries)")
