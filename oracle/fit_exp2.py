"""Fit the polynomial p(f) ~ 2**f on [0, 1] used by the contract exponential.

Test infrastructure: this script only produces the coefficient table that the
oracle (oracle/wh_oracle.c) and the HIP kernels (whallm_amd/csrc/wh_common.h)
both hard-code.  Method: Lawson's minimax iteration on the relative error of a degree-6
polynomial with p(0) = 1 fixed, in float64, then each coefficient is rounded to
float32 and the float32 Horner evaluation (with fused multiply-adds) is checked
on a dense grid.  Run:  python oracle/fit_exp2.py
"""
import numpy as np

DEG = 6


def fit(deg=DEG, iters=400):
    """Lawson's algorithm: iteratively reweighted least squares converging to
    the minimax fit of the relative error p(f)/2^f - 1, with p(0) = 1 fixed."""
    grid = 0.5 - 0.5 * np.cos(np.linspace(0.0, np.pi, 4001))
    w2 = 2.0 ** grid
    V = np.stack([grid ** k / w2 for k in range(1, deg + 1)], axis=1)
    rhs = 1.0 - 1.0 / w2
    lw = np.full(grid.shape, 1.0 / grid.size)
    for _ in range(iters):
        sw = np.sqrt(lw)
        c, *_ = np.linalg.lstsq(V * sw[:, None], rhs * sw, rcond=None)
        err = np.abs(V @ c - rhs)
        lw = lw * err
        lw /= lw.sum()
    fine = np.linspace(0.0, 1.0, 400001)
    p = 1.0 + sum(c[k - 1] * fine ** k for k in range(1, deg + 1))
    return np.concatenate([[1.0], c]), float(np.max(np.abs(p / 2.0 ** fine - 1.0)))


def horner_f32(coef32, f):
    f = np.asarray(f, dtype=np.float32)
    p = np.full_like(f, coef32[-1])
    for ck in coef32[-2::-1]:
        # fused multiply-add in float32: compute in float64 then round once
        p = (p.astype(np.float64) * f.astype(np.float64) + np.float64(ck)).astype(np.float32)
    return p


if __name__ == "__main__":
    coef, err = fit()
    coef32 = coef.astype(np.float32)
    f = np.linspace(0.0, 1.0, 1 << 22, endpoint=False, dtype=np.float64).astype(np.float32)
    p = horner_f32(coef32, f)
    rel = np.abs(p.astype(np.float64) / np.exp2(f.astype(np.float64)) - 1.0)
    print("minimax max rel err (float64 coefficients): %.3e" % err)
    print("float32 Horner max rel err on grid: %.3e (%.2f ulp of 2^-23)" % (rel.max(), rel.max() / 2 ** -23))
    for k, ck in enumerate(coef32):
        print("C%d = %s  /* %s */" % (k, np.float32(ck).hex() if hasattr(np.float32(ck), 'hex') else float(ck), repr(float(ck))))
    print("hex floats:", ", ".join(float(c).hex() for c in coef32))
