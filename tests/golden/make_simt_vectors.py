"""Write the projection / router / MoE known-answer vectors of the reference's
GPU tests (tests/qwen35_simt.rs:93-434) as fixtures.

The reference ships no expected outputs for these tests, only a host oracle
inside the test file (`dot_width`, tests/qwen35_simt.rs:99-116) and an input
generator (`values`, :118-127). Both are transcribed here from the test's
text (the reference is read, not run) with IEEE binary32 scalar arithmetic,
and the outputs they define for the test's own shapes are stored in
simt_known_answers.json. The checker (oracle/) and the GPU kernels are then
compared against these fixtures.

Usage: python tests/golden/make_simt_vectors.py
"""
from __future__ import annotations

import json
import os

import numpy as np

F = np.float32
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "simt_known_answers.json")


def f32_to_bf16(x) -> int:
    """src/weights.rs:213-221."""
    u = int(np.array([x], dtype=np.float32).view(np.uint32)[0])
    if np.isnan(F(x)):
        return ((u >> 16) | 0x0040) & 0xFFFF
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF


def bf16_to_f32(b: int):
    return np.array([b << 16], dtype=np.uint32).view(np.float32)[0]


def values(n: int, seed: int) -> list[int]:
    """tests/qwen35_simt.rs:118-127 (integer division as in Rust usize)."""
    out = []
    for i in range(n):
        scale = F(2.0) ** F(((i * seed // 37) % 17) - 8)
        v = (F((i * seed) % 37) - F(18.0)) / F(64.0) * scale
        out.append(f32_to_bf16(F(v)))
    return out


def dot_width(a: list[int], b: list, width: int):
    """tests/qwen35_simt.rs:99-116 with F32 scalars (no fused multiply-add)."""
    sums = [F(0.0)] * width
    pairs = len(a) // 2
    for lane in range(width):
        low, high = F(0.0), F(0.0)
        for pair in range(lane, pairs, width):
            low = F(low + F(bf16_to_f32(a[2 * pair]) * F(b[2 * pair])))
            high = F(high + F(bf16_to_f32(a[2 * pair + 1]) * F(b[2 * pair + 1])))
        sums[lane] = F(low + high)
    shift = 1
    while (width >> shift) >= 1:
        stride = width >> shift
        for lane in range(stride):
            sums[lane] = F(sums[lane] + sums[lane + stride])
        shift += 1
    return sums[0]


def as_f32(bits: list[int]) -> list:
    return [bf16_to_f32(b) for b in bits]


def random_bf16(n: int, seed: int) -> list[int]:
    """Deterministic BF16 words with mixed signs and magnitudes (xorshift32)."""
    state = (seed * 2654435761) & 0xFFFFFFFF or 1
    out = []
    for _ in range(n):
        state ^= (state << 13) & 0xFFFFFFFF
        state ^= state >> 17
        state ^= (state << 5) & 0xFFFFFFFF
        mant = F((state & 0xFFFF) / 65536.0 - 0.5)
        scale = F(2.0) ** F(((state >> 16) % 9) - 4)
        out.append(f32_to_bf16(F(mant * scale)))
    return out


def main() -> None:
    fixtures = {"source": "tests/qwen35_simt.rs:93-434 (hellas-ai/catena-models)",
                "projections": [], "grouped": [], "router": [], "moe_down": []}
    # projections_match_reference (:129-215)
    for k, n in [(2, 1), (62, 3), (64, 5), (66, 17), (254, 7), (256, 4), (258, 5), (2048, 33)]:
        x = values(k, 7)
        w = values(k * n, 13)
        residual = values(n, 11)
        project, resid = [], []
        for row in range(n):
            wr = as_f32(w[row * k:(row + 1) * k])
            g32 = dot_width(x, wr, 32)
            g64 = dot_width(x, wr, 64)
            project.append(f32_to_bf16(g32))
            resid.append(f32_to_bf16(F(bf16_to_f32(f32_to_bf16(g64)) + bf16_to_f32(residual[row]))))
        fixtures["projections"].append(
            {"k": k, "n": n, "x_seed": 7, "w_seed": 13, "residual_seed": 11,
             "project": project, "residual": resid})
    # grouped projections (:223-258)
    x = values(3 * 256, 7)[:256]
    for bank, n in enumerate([126, 66, 66]):
        w = values(n * 256, 11 + bank * 2)
        out = [f32_to_bf16(dot_width(x, as_f32(w[r * 256:(r + 1) * 256]), 256)) for r in range(n)]
        fixtures["grouped"].append({"rows": n, "w_seed": 11 + bank * 2, "out": out})
    # F32 router (:259-308): weights ((i*13 % 37) - 18) / 64, shared row 0.125
    weights = [(F((i * 13) % 37) - F(18.0)) / F(64.0) for i in range(4 * 256)]
    shared = [F(0.125)] * 256
    for token in range(3):
        xt = values(3 * 256, 7)[token * 256:(token + 1) * 256]
        row_bits = []
        for row in range(5):
            wr = weights[row * 256:(row + 1) * 256] if row < 4 else shared
            row_bits.append(int(np.array([dot_width(xt, wr, 32)], dtype=np.float32).view(np.uint32)[0]))
        fixtures["router"].append({"token": token, "logit_bits": row_bits})
    # MoE down (:390-434): experts [1, 3], I = 66, SI = 258, H = 256
    act = values(132 + 258, 19)
    down = values(4 * 256 * 66, 11)
    sd = values(256 * 258, 17)
    residual = values(256, 5)
    out = []
    for row in range(256):
        w = []
        for e in [1, 3]:
            w += as_f32(down[(e * 256 + row) * 66:(e * 256 + row + 1) * 66])
        routed = f32_to_bf16(F(dot_width(act[:132], w, 32) + bf16_to_f32(residual[row])))
        sh = f32_to_bf16(dot_width(act[132:], as_f32(sd[row * 258:(row + 1) * 258]), 32))
        out.append(f32_to_bf16(F(bf16_to_f32(routed) + bf16_to_f32(sh))))
    fixtures["moe_down"].append({"experts": [1, 3], "hidden": 256, "intermediate": 66,
                                 "shared": 258, "activation_seed": 19, "down_seed": 11,
                                 "shared_seed": 17, "residual_seed": 5, "out": out})
    # F32 values of the same host oracle on inputs that exercise rounding:
    # the BF16-rounded outputs above do not depend on the tree shape for the
    # test's nearly exactly-summable inputs, these F32 bits do.
    fixtures["random_dots"] = []
    for pairs, seed in [(1024, 1), (2048, 2), (256, 3), (129, 4)]:
        x, w = random_bf16(2 * pairs, seed), random_bf16(2 * pairs, seed + 100)
        entry = {"pairs": pairs, "seed": seed}
        for width in (32, 64, 256):
            v = dot_width(x, as_f32(w), width)
            entry[f"w{width}"] = int(np.array([v], dtype=np.float32).view(np.uint32)[0])
        fixtures["random_dots"].append(entry)
    with open(OUT, "w") as f:
        json.dump(fixtures, f, separators=(",", ":"))
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
