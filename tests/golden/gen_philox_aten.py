"""Writes tests/golden/philox_aten.npz: Philox4x32-10 outputs computed by
ATen's PhiloxRNGEngine.h (torch/include/ATen/core/PhiloxRNGEngine.h), an
implementation independent of this repository's oracle and kernels.

ATen's engine uses key = (seed_lo, seed_hi) and
counter = (offset_lo, offset_hi, subsequence_lo, subsequence_hi); its first
four outputs are the four words of Philox4x32-10(counter, key).  The sampler's
stream is counter = (node_lo, node_hi, draw, 0), key = (seed_lo, seed_hi), i.e.
offset = node and subsequence = draw.

Run:  python tests/golden/gen_philox_aten.py   (needs g++ and torch headers)
"""
import os
import subprocess
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

PROG = r'''
#include <ATen/core/PhiloxRNGEngine.h>
#include <cstdio>
#include <cstdint>
int main() {
  unsigned long long seed, off, sub;
  while (std::scanf("%llu %llu %llu", &seed, &off, &sub) == 3) {
    at::philox_engine e(seed, sub, off);
    uint32_t a = e(), b = e(), c = e(), d = e();
    std::printf("%u %u %u %u\n", a, b, c, d);
  }
  return 0;
}
'''


def main():
    import torch.utils.cpp_extension as ce
    inc = ce.include_paths()
    rng = np.random.default_rng(20240601)
    cases = [(0, 0, 0), (42, 0, 0), (42, 1, 0), (42, 0, 1), (42, 110_999_999, 14),
             (2**64 - 1, 2**64 - 1, 2**32 - 1), (42, 2**32, 3), (42, 2**32 - 1, 7)]
    for _ in range(56):
        cases.append((int(rng.integers(0, 2**63)), int(rng.integers(0, 2**40)),
                      int(rng.integers(0, 2**32))))
    for node in range(0, 200, 7):
        for draw in range(0, 64, 9):
            cases.append((42, node, draw))
    with tempfile.TemporaryDirectory() as td:
        src = os.path.join(td, "p.cpp")
        exe = os.path.join(td, "p")
        with open(src, "w") as f:
            f.write(PROG)
        cmd = ["g++", "-O1", "-std=c++17", src, "-o", exe] + [f"-I{p}" for p in inc]
        subprocess.run(cmd, check=True)
        inp = "\n".join(f"{s} {o} {d}" for s, o, d in cases) + "\n"
        out = subprocess.run([exe], input=inp, capture_output=True, text=True, check=True).stdout
    words = np.array([[int(x) for x in ln.split()] for ln in out.strip().splitlines()], np.uint64)
    seeds = np.array([c[0] for c in cases], np.uint64)
    nodes = np.array([c[1] for c in cases], np.uint64)
    draws = np.array([c[2] for c in cases], np.uint64)
    np.savez(os.path.join(HERE, "philox_aten.npz"), seed=seeds, node=nodes, draw=draws,
             words=words.astype(np.uint32))
    print(f"wrote {len(cases)} vectors")


if __name__ == "__main__":
    main()
