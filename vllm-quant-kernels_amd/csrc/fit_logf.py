"""Derives the polynomial used by vqk_logf (csrc/vqk_math.h and oracle/vqk_oracle.c).

log(1+f) on f in [sqrt(1/2)-1, sqrt(2)-1] is written as f - f^2/2 + f^3 * P(f); P is a
degree-DEG polynomial fitted to (log1p(f) - f + f^2/2) / f^3 by least squares on
Chebyshev nodes in float64, then each coefficient is rounded to float32.  Running
this file prints the coefficients and the worst error (in float32 ulps) of the float32
evaluation, done with the same fma order as the kernels, over a dense sweep.

The polynomial is this project's own fit (no library constants are reused); the
kernel and the oracle evaluate it with identical IEEE float32 operations so the noise
they produce is bit-identical.
"""
import numpy as np

DEG = 7
LO, HI = np.sqrt(0.5) - 1.0, np.sqrt(2.0) - 1.0


def fit(deg=DEG):
    n = 4000
    t = np.cos(np.pi * (np.arange(n) + 0.5) / n)
    f = LO + (HI - LO) * (t + 1) / 2
    f = f[np.abs(f) > 1e-3]
    r = (np.log1p(f) - f + 0.5 * f * f) / (f ** 3)
    V = np.vander(f, deg + 1, increasing=True)
    c, *_ = np.linalg.lstsq(V, r, rcond=None)
    return c.astype(np.float32)


def eval_f32(x, c):
    """float32 evaluation with the kernel's operation order (fma emulated in float64,
    which is exact for a single fma of float32 operands up to the final rounding)."""
    x = np.asarray(x, np.float32)
    bits = x.view(np.uint32)
    e = ((bits >> 23) & 0xFF).astype(np.int32) - 127
    mb = bits & 0x7FFFFF
    big = mb > 0x3504F3
    m = np.where(big, (mb | 0x3F000000), (mb | 0x3F800000)).astype(np.uint32).view(np.float32)
    e = np.where(big, e + 1, e)
    f = (m - np.float32(1.0)).astype(np.float32)

    def fma(a, b, cc):
        return (a.astype(np.float64) * b.astype(np.float64) + cc.astype(np.float64)).astype(np.float32)

    p = np.full_like(f, c[-1])
    for ci in c[-2::-1]:
        p = fma(p, f, np.full_like(f, ci))
    f2 = (f * f).astype(np.float32)
    f3 = (f2 * f).astype(np.float32)
    t = fma(f3, p, (np.float32(-0.5) * f2).astype(np.float32))
    y = (f + t).astype(np.float32)
    ef = e.astype(np.float32)
    y = fma(ef, np.full_like(f, np.float32(1.42860677e-06)), y)
    y = fma(ef, np.full_like(f, np.float32(0.693145752)), y)
    return y


def ulp_err(x, c):
    y = eval_f32(x, c).astype(np.float64)
    ref = np.log(np.asarray(x, np.float64))
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    return np.abs(y - ref) / ulp


if __name__ == "__main__":
    c = fit()
    print("coefficients (float32):")
    for i, ci in enumerate(c):
        print(f"  c{i} = {float(ci)!r}f  /* 0x{np.float32(ci).view(np.uint32):08X} */")
    xs = np.concatenate([
        np.linspace(0.5, 2.0, 2_000_001, dtype=np.float32),
        np.geomspace(1e-7, 100.0, 2_000_001).astype(np.float32),
        (1.0 - np.arange(1, 200000, dtype=np.float64) * 2.0 ** -24).astype(np.float32),
    ])
    xs = xs[xs != 1.0]
    err = ulp_err(xs, c)
    print(f"max error {err.max():.3f} ulp over {xs.size} points")
