"""Writes rng_vectors.json: closed-form values of the reference's xorshift64 `Rng`
(crates/bfi-runtime/src/sample.rs:441-460) and `slot_rng` (engine/spec.rs:185-187),
computed here with Python integers, independently of the C oracle. The entries for seeds
0/1/7/42/12345 and slot_rng(7, 9) reproduce values derived by hand from the reference."""
import json
import os

import numpy as np

M = (1 << 64) - 1


def nxt(x):
    if x == 0:
        x = 0x9E3779B97F4A7C15
    x ^= (x << 13) & M
    x ^= x >> 7
    x ^= (x << 17) & M
    return x


def u_of(word):
    return float(np.float32(word >> 40) / np.float32(1 << 24))


def stream(seed, n):
    words, us, x = [], [], seed
    for _ in range(n):
        x = nxt(x)
        words.append(hex(x))
        us.append(u_of(x))
    return words, us


def main():
    seeds = [0, 1, 7, 42, 12345, 0x8000000000000005, M, 0x0123456789ABCDEF]
    out = {"rng": [], "slot_rng": []}
    for s in seeds:
        w, u = stream(s, 6)
        out["rng"].append({"seed": hex(s), "words": w, "u": u})
    for seed, plen in [(7, 9), (0, 0), (42, 1000), (M, 3)]:
        s = seed ^ 0xA0761D6478BD642F ^ ((plen * 0x9E3779B97F4A7C15) & M)
        w, u = stream(s, 4)
        out["slot_rng"].append({"seed": hex(seed), "prompt_len": plen, "state": hex(s), "u": u})
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "rng_vectors.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
