"""Writes tests/golden/needle3_golden.npz: the reference's own numpy forward
of Needle 3 (tools/golden.py) on seeded random-init archives.

Runs in the build container only (it imports the reference from
/root/reference, which the GPU box does not have; .gpurunignore keeps this
script off it).  Only the vectors it writes travel with the tests.

The reference holds its engine to this forward on the real model at cosine
> 0.99995 with the same argmax (tests/Needle.Tests/ParityTests.cs:55-57).  Its
forward dequantizes every weight to float and multiplies float activations
(tools/golden.py:109-124, 194-232), so it does not model the engine's int8
activations (Quant.Prepare per 128-group); the tests that read these vectors
state the bounds that follow from that.

Per case the file holds:
  <case>_seed       the archive seed: needle_cs_amd.archive.needle3_archive(NEEDLE3, seed)
  <case>_sha256     the archive's sha256 (the tests refuse a drifted generator)
  <case>_tokens     int32 [n], drawn from numpy's default_rng(seed)
  <case>_logits     float32 [vocab], Model.forward(tokens): the last token's logits
  <case>_engram     int32 [n][tables], engram_indices(tokens, orders, 3, slots)
and for the cases with layer states (dump=...):
  <case>_x0         float32 [dim], the last token's embedding (golden.py:253)
  <case>_deltas     float16 [layers][4][dim], the last token's stream after
                    layer l minus before it (the streamNN dumps, golden.py:266-267;
                    before layer 0 every lane holds x0)
"""
from __future__ import annotations

import hashlib
import importlib.util
import os
import pathlib
import sys
import tempfile
import time

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent.parent
REFERENCE_GOLDEN = pathlib.Path("/root/reference/tools/golden.py")
OUT = HERE / "needle3_golden.npz"

# (case, archive seed, tokens, with per-layer states)
CASES = [("short", 11, 24, True), ("prompt", 12, 40, True), ("window", 13, 1100, False)]


def load_reference():
    spec = importlib.util.spec_from_file_location("needle_reference_golden", REFERENCE_GOLDEN)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main() -> None:
    sys.path.insert(0, str(ROOT))
    from needle_cs_amd.archive import NEEDLE3, needle3_archive

    ref = load_reference()
    out = {}
    for case, seed, n, states in CASES:
        t0 = time.time()
        archive = needle3_archive(NEEDLE3, seed)
        with tempfile.TemporaryDirectory() as tmp:
            path = os.path.join(tmp, "model.cact")
            with open(path, "wb") as f:
                f.write(archive)
            model = ref.Model(ref.Cact(path))
            tokens = np.random.default_rng(seed).integers(0, NEEDLE3["vocab"], n).astype(np.int64)
            dump = pathlib.Path(tmp) if states else None
            logits = model.forward(tokens, dump=dump)[0].astype(np.float32)
            if states:
                dim, layers = NEEDLE3["dim"], NEEDLE3["layers"]
                x0 = np.fromfile(dump / "x0.bin", np.float32).reshape(n, dim)[-1]
                prev = np.repeat(x0[None, :], 4, 0)
                deltas = []
                for l in range(layers):
                    s = np.fromfile(dump / f"stream{l:02d}.bin", np.float32).reshape(n, 4, dim)[-1]
                    deltas.append(s - prev)
                    prev = s
                out[f"{case}_x0"] = x0
                out[f"{case}_deltas"] = np.stack(deltas).astype(np.float16)
        out[f"{case}_seed"] = np.int64(seed)
        out[f"{case}_sha256"] = np.array(hashlib.sha256(archive).hexdigest())
        out[f"{case}_tokens"] = tokens.astype(np.int32)
        out[f"{case}_logits"] = logits
        out[f"{case}_engram"] = ref.engram_indices(tokens, list(NEEDLE3["orders"]), 3,
                                                   NEEDLE3["engram_slots"]).astype(np.int32)
        print(f"{case}: seed {seed}, {n} tokens, argmax {int(logits.argmax())}, {time.time() - t0:.1f} s", flush=True)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
