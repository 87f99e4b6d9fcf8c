"""Writes sampler_vectors.json: outputs of the reference's own Gaussian-noise
generator (src/sampler/sampler.cpp:37-61, fill_gaussian_noise), compiled from
the reference sources into oracle/_ref by `make -C oracle ref`.

Each case stores (seed, stream, count) and the float32 bit patterns of the
output, so the oracle's restatement can be checked bit for bit where the
reference checkout (and with it oracle/_ref) is absent.

    python tests/golden/gen_sampler_vectors.py
"""

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))

import oracle as O  # noqa: E402

# (seed, stream, count): the reference smoke test's seed/stream (tools/sampler_smoke.cpp:43, :62),
# a 64-bit stream, odd counts (the last Box-Muller pair is half used), and the
# benchmark workload's per-block seeds.
CASES = [
    (666, 7, 33),
    (666, 8, 16),
    (666, (1 << 32) + 7, 16),
    (667, 7, 16),
    (20260823, 0, 17),
    (20260824, 1, 24),
    (20260825, 3, 32),
    (0, 0, 5),
    (4294967295, (1 << 64) - 1, 9),
]


def main() -> None:
    ref = O.ref_sampler()
    if ref is None:
        raise SystemExit("oracle/_ref/libref_sampler.so missing: run `make -C oracle ref` with the reference present")
    out = []
    for seed, stream, count in CASES:
        buf = np.zeros(count + 1, np.float32)
        if ref.ref_fill_gaussian_noise(buf.ctypes.data, count, seed, stream) != 0:
            raise SystemExit(f"reference generator refused {(seed, stream, count)}")
        out.append({"seed": seed, "stream": stream, "count": count,
                    "bits": [f"{b:08x}" for b in buf[:count].view(np.uint32).tolist()]})
    path = os.path.join(HERE, "sampler_vectors.json")
    with open(path, "w") as f:
        json.dump({"generator": "src/sampler/sampler.cpp fill_gaussian_noise (compiled reference)", "cases": out}, f,
                  indent=1)
    print(f"wrote {path} ({len(out)} cases)")


if __name__ == "__main__":
    main()
