"""Per-stage timeline of the persistent decode run (diagnostic).

The run records, for one chosen decode step, every block's gather completion
and publication of each stage plus points inside layer 5's stages, as
s_memrealtime stamps (100 MHz), when the library is built with

    make -C unlimitedocr.c_amd -B EXTRA="-DUOCR_RUN_TIMELINE -DUOCR_RUN_TL_NOWAIT"

(UOCR_RUN_TL_NOWAIT leaves out the one stamp that waits for a wavefront's
loads).  That build is slower than the product (about 1-2%) and replaces the
in-tree library: rebuild with a plain `make -C unlimitedocr.c_amd -B`
afterwards.  Run on the GPU from the repository root:

    python unlimitedocr.c_amd/run_timeline.py [--step 20] [--out timeline.npy]

It decodes 64 greedy steps of the config-5 prompt (900 image rows + 31 text
ids + BOS, synthetic Q4 model) and prints, for layers 1-10 averaged, each
stage's hand-off (the previous stage's last publish to the stage's median
block having its inputs), compute (median inputs to median publish) and tail
(median to last publish), then the GU stage's inner points of layer 5.
"""
from __future__ import annotations

import argparse
import ctypes as ct
import os
import sys
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parent))
os.environ.setdefault("UOCR_HIP_RUN", "1")
import uocr  # noqa: E402

EVENTS = 256  # stamps per block
STAGES = ["QKV", "ATT", "O", "GU", "DN"]
# layer 5 inner points: event 128 + k
GU_POINTS = [(18, "z gathered"), (22, "z summed"), (23, "top-6 chosen"), (33, "first poll round for a issued"),
             (10, "expert rows issued"), (24, "a gathered"), (15, "block barrier after a"), (16, "norm of a"),
             (11, "dots and router quarter"), (19, "mids published"), (20, "DN rows issued")]


def stage(h: np.ndarray, t0: int, c: int, blocks=None):
    g, e = h[:, 2 * c], h[:, 2 * c + 1]
    act = (g > 0) & (e > 0)
    if blocks is not None:
        sel = np.zeros(h.shape[0], bool)
        sel[list(blocks)] = True
        act &= sel
    return (g[act] - t0) * 0.01, (e[act] - t0) * 0.01


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--step", type=int, default=20, help="decode step to record (< 64)")
    ap.add_argument("--out", default=None, help="save the raw stamps ([256][256] u64) to this .npy file")
    args = ap.parse_args()
    lib = uocr.load_library()
    if not hasattr(lib, "uocr_run_timeline"):
        print("the library was not built with -DUOCR_RUN_TIMELINE (see this script's docstring)", file=sys.stderr)
        return 2
    lib.uocr_run_timeline.argtypes = [ct.c_void_p, ct.c_int]
    lib.uocr_run_timeline.restype = ct.c_int

    model = uocr.synth_model(uocr.QPROFILE_Q4, 7)
    eng = uocr.Engine.from_memory(model, backend="hip", max_prompt_tokens=1024, max_gen_tokens=600)
    rng = np.random.default_rng(5)
    ids = np.concatenate([[0], np.full(900, 128815), rng.integers(2, 128000, 31)]).astype(np.int32)
    mask = (ids == 128815).astype(np.uint8)
    rows = rng.standard_normal((900, 1280)).astype(np.float16)

    buf = uocr.DeviceBuffer(256 * EVENTS * 8)
    buf.zero()
    if lib.uocr_run_timeline(ct.c_void_p(buf.ptr), args.step) != 0:
        print("uocr_run_timeline failed", file=sys.stderr)
        return 1
    steps = 64
    _, _, _, dec_ms = eng.generate_embeddings(ids, mask, rows, max_new_tokens=steps, flags=uocr.GEN_IGNORE_EOS)
    lib.uocr_run_timeline(None, -1)
    eng.close()
    h = buf.download(np.uint64).reshape(256, EVENTS).astype(np.int64)
    if args.out:
        np.save(args.out, h)
    start = h[:, 127][h[:, 127] > 0]
    if start.size == 0:
        print("no stamps recorded (step beyond the generation?)", file=sys.stderr)
        return 1
    t0 = int(start.min())
    print(f"decode {dec_ms:.2f} ms for {steps} tokens ({steps / dec_ms * 1e3:.0f} tok/s in this build); step {args.step}")

    print("\nstage  hand-off  compute  tail   (us, layers 1-10 averaged, medians over the stage's blocks)")
    total = 0.0
    for s, name in enumerate(STAGES):
        vals = []
        for layer in range(1, 11):
            c = 1 + 5 * layer + s
            g, e = stage(h, t0, c)
            _, pe = stage(h, t0, c - 1)
            if g.size and e.size and pe.size:
                vals.append((np.median(g) - pe.max(), np.median(e) - np.median(g), e.max() - np.median(e)))
        if vals:
            v = np.mean(np.array(vals), axis=0)
            total += float(v.sum())
            print(f"{name:5s} {v[0]:8.2f} {v[1]:8.2f} {v[2]:6.2f}")
    print(f"per layer {total:.2f} us")

    att_last = stage(h, t0, 1 + 5 * 5 + 1)[1].max()
    o_last = stage(h, t0, 1 + 5 * 5 + 2)[1].max()
    print(f"\nlayer 5 GU, us after the attention stage's last publish (the O stage's last publish at {o_last - att_last:.2f}):")
    for k, label in GU_POINTS:
        col = h[:, 128 + k]
        a = col > 0
        if a.any():
            v = (col[a] - t0) * 0.01 - att_last
            print(f"  {label:30s} median {np.median(v):6.2f}  last {v.max():6.2f}  ({int(a.sum())} blocks)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
