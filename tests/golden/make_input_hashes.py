"""Writes tests/golden/input_sha256.json: the SHA-256 of every seeded input buffer bench.py generates
with kriya_q4.synth (configs 0, 1, 2 and 4 at full size), so that any host -- this one, the GPU box --
can check that it regenerates byte-identical inputs.  Config 3's model weights come from torch's device
generator and are not listed.

Run: python tests/golden/make_input_hashes.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "kriya-rt_amd"))

from kriya_q4 import synth  # noqa: E402


def inputs():
    """(name, array) of every seeded input of bench.py's configurations 0, 1, 2 and 4."""
    H, I, E, MI = synth.HIDDEN, synth.INTER, 60, 1408
    yield "cfg0_w", synth.q4_weight(I, H, 0)
    yield "cfg0_x", (synth.bf16_normal((1, H), 1),)
    for t, (n, k) in zip((1001, 1002, 1003), ((I, H), (I, H), (H, I))):
        yield f"cfg1_w{t}", synth.q4_weight(n, k, t)
    for B in (1, 4, 16):
        yield f"cfg1_h_B{B}", (synth.bf16_normal((B, H), 1010 + B),)
    shapes = [(H, H), (256, H), (256, H), (H, H), (I, H), (I, H), (H, I)]
    for i, (n, k) in enumerate(shapes):
        yield f"cfg2_w{2000 + i}", synth.q4_weight(n, k, 2000 + i)
    yield "cfg2_x", (synth.bf16_normal((512, H), 2100),)
    for t, (n, k) in zip((4001, 4002, 4003), ((E * MI, H), (E * MI, H), (E * H, MI))):
        yield f"cfg4_w{t}", synth.q4_weight(n, k, t)
    for T in (1, 64):
        yield f"cfg4_x_T{T}", (synth.bf16_normal((T, H), 4004),)
        yield f"cfg4_logits_T{T}", (synth.f32_normal((T, E), 4005),)


def digest(arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(a.tobytes())
    return h.hexdigest()


def main():
    out = {name: digest(arrays) for name, arrays in inputs()}
    with open(os.path.join(HERE, "input_sha256.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"wrote {len(out)} digests")


if __name__ == "__main__":
    main()
