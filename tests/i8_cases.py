"""Inputs that tell the int8 quantizer's reciprocal rule apart.

q4k_quantize_x_q8 (stratum_q4k_neon.h:262-276) and q6k_quantize_x_q8_g16
(stratum_q6k_neon.h:117-133) round x * inv with inv = fl(1 / scale), not
x / scale.  The two round to different integers only when x / scale lies
within a few binary32 ulps of a half-integer; reciprocal_groups finds such
x by a seeded search and returns them in groups whose largest |x| fixes the
scale, so a quantizer that divides instead fails on them.
"""
import numpy as np

f32 = np.float32


def _step(v, n):
    for _ in range(abs(n)):
        v = np.nextafter(v, f32(np.inf) if n > 0 else f32(-np.inf), dtype=f32)
    return v


def reciprocal_cases(n, seed=4242):
    """n triples (amax, x, q): |x| <= amax, scale = fl(amax / 127), inv =
    fl(1 / scale); q = rne(fl(x * inv)) differs from rne(fl(x / scale))."""
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        amax = f32(r.uniform(0.05, 20.0))
        scale = f32(amax / f32(127.0))
        inv = f32(f32(1.0) / scale)
        k = int(r.integers(-126, 126))
        base = f32((k + 0.5) * np.float64(scale))
        for d in range(-4, 5):
            x = _step(base, d)
            if abs(x) > amax:
                continue
            q_mul, q_div = np.rint(f32(x * inv)), np.rint(f32(x / scale))
            if q_mul != q_div:
                out.append((amax, x, int(q_mul)))
                break
    return out


def reciprocal_groups(G, n, seed=4242):
    """x of n groups of G values (group g: amax at 0, the case's x at 1,
    zeros after) and the expected int8 value at position 1 of each group."""
    cases = reciprocal_cases(n, seed)
    x = np.zeros(n * G, f32)
    want = np.empty(n, np.int32)
    for g, (amax, xv, q) in enumerate(cases):
        x[g * G] = amax
        x[g * G + 1] = xv
        want[g] = q
    return x, want
