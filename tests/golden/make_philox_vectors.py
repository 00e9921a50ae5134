"""Writes tests/golden/philox4x32_10.json: Philox4x32-10 words computed by rocRAND's engine
(/opt/rocm/include/rocrand/rocrand_philox4x32_10.h, built here for the host with hipcc), an
implementation independent of the oracle's, for the oracle's known-answer test.

Cases: the three known-answer inputs of the Random123 distribution (counter 0 / key 0, all ones,
the pi digits), a grid of counters and keys with carries in every word, and the blocks of a
small dropout layout.  Run in an image with ROCm's headers and hipcc:

    python tests/golden/make_philox_vectors.py
"""

import json
import random
import subprocess
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent

PROGRAM = r"""
#include <cstdio>
#include <rocrand/rocrand_philox4x32_10.h>

// rocRAND keeps its ten rounds protected; a derived class exposes them unchanged.
struct Engine : rocrand_device::philox4x32_10_engine {
    uint4 words(uint4 c, uint2 k) { return this->ten_rounds(c, k); }
};

int main() {
    Engine e;
    unsigned c0, c1, c2, c3, k0, k1;
    while (std::scanf("%x %x %x %x %x %x", &c0, &c1, &c2, &c3, &k0, &k1) == 6) {
        const uint4 w = e.words(uint4{c0, c1, c2, c3}, uint2{k0, k1});
        std::printf("%08x %08x %08x %08x\n", w.x, w.y, w.z, w.w);
    }
    return 0;
}
"""


def cases():
    out = [
        ((0, 0, 0, 0), (0, 0)),
        ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF)),
        ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0)),
    ]
    rng = random.Random(20261202)
    for _ in range(40):
        out.append((tuple(rng.getrandbits(32) for _ in range(4)), (rng.getrandbits(32), rng.getrandbits(32))))
    # dropout layout blocks: n = row * ceil(S/4) + s/4 split over (c0, c1), offset over (c2, c3)
    for n, offset, seed in [(0, 0, 1), (1, 0, 1), (5, 0, 0x123456789ABCDEF0), (2 ** 32 + 7, 3, 42),
                            (2 ** 40 + 1, 2 ** 33 + 5, 2 ** 64 - 1)]:
        out.append(((n & 0xFFFFFFFF, n >> 32, offset & 0xFFFFFFFF, offset >> 32), (seed & 0xFFFFFFFF, seed >> 32)))
    return out


def main():
    cs = cases()
    with tempfile.TemporaryDirectory() as d:
        src, exe = Path(d) / "philox.cpp", Path(d) / "philox"
        src.write_text(PROGRAM)
        subprocess.run(["/opt/rocm/bin/hipcc", "-x", "hip", "--offload-arch=gfx950", "-O1", "-I/opt/rocm/include",
                        str(src), "-o", str(exe)], check=True)
        stdin = "".join("%x %x %x %x %x %x\n" % (*c, *k) for c, k in cs)
        res = subprocess.run([str(exe)], input=stdin, capture_output=True, text=True, check=True).stdout.split("\n")
    vectors = []
    for (c, k), line in zip(cs, res):
        vectors.append({"counter": list(c), "key": list(k), "words": [int(x, 16) for x in line.split()]})
    lines = ",\n  ".join(json.dumps(v) for v in vectors)
    (HERE / "philox4x32_10.json").write_text(
        '{"source": "rocRAND philox4x32_10_engine::ten_rounds",\n "vectors": [\n  ' + lines + "\n ]\n}\n")
    print(f"wrote {len(vectors)} vectors")


if __name__ == "__main__":
    main()
