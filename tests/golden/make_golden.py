"""Writes tests/golden/rmsnorm_residual_golden.json — independent truth for the oracle and kernels.

Pure Python (no NumPy, no torch, no reference import): inputs are float32 (or bfloat16)
representable numbers from a seeded `random.Random`; expected values are computed with exact
rationals and 60-digit decimals:
  forward   h = x + residual; inv_rms = 1/sqrt(sum(h^2)/D + eps32); y = h*inv_rms*w
            (python/velograd/kernels/fused.py:39-45, eps rounded to float32 as NumPy does when a
            Python float meets a float32 array)
  backward  dL/dh and dL/dw of L = sum(g * y) by central finite differences of the forward
            above (step 1e-20), NOT by the analytic formula of fused.py:58-65, so the golden
            backward pins that formula (and its `normed_input = h * inv_rms` convention).
Cases: the reference's own known answers (Rust RMSNorm test tests/core_engine_tests.rs:243-247,
gradcheck inputs tests/test_velograd_beast.py:121 and tests/test_velograd_omnibus_grand_master.py:125),
seeded random rows, bfloat16-representable rows, and special rows (zero, constant, outlier).

Run:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import os
import random
import struct
from decimal import Decimal, getcontext
from fractions import Fraction

getcontext().prec = 60
FD_STEP = Decimal("1e-20")
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "rmsnorm_residual_golden.json")


def f32(v: float) -> float:
    return struct.unpack("<f", struct.pack("<f", v))[0]


def bf16(v: float) -> float:
    """Round a float32-representable value to bfloat16, nearest-even."""
    u = struct.unpack("<I", struct.pack("<f", f32(v)))[0]
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return struct.unpack("<f", struct.pack("<I", u))[0]


def dec(v) -> Decimal:
    if isinstance(v, Fraction):
        return Decimal(v.numerator) / Decimal(v.denominator)
    return Decimal(Fraction(v).numerator) / Decimal(Fraction(v).denominator)


def forward_row(h, w, eps32):
    """Exact forward of one row given h (list of Decimal): returns (y, inv_rms)."""
    d = len(h)
    ms = sum(v * v for v in h) / Decimal(d)
    inv = Decimal(1) / (ms + dec(eps32)).sqrt()
    y = [v * inv * (dec(w[j]) if w is not None else Decimal(1)) for j, v in enumerate(h)]
    return y, inv


def loss_row(h, w, g, eps32):
    y, _ = forward_row(h, w, eps32)
    return sum(dec(g[j]) * y[j] for j in range(len(h)))


def make_case(name, x, res, w, g, eps, note):
    eps32 = f32(eps)
    rows = len(x)
    d = len(x[0])
    out = {"name": name, "note": note, "eps": eps, "rows": rows, "dim": d,
           "x": x, "residual": res, "weight": w, "grad_y": g}
    ys, hs, invs = [], [], []
    dxs = []
    dw = [Decimal(0)] * d if w is not None else None
    for r in range(rows):
        h = [dec(x[r][j]) + (dec(res[r][j]) if res is not None else Decimal(0)) for j in range(d)]
        y, inv = forward_row(h, w, eps32)
        ys.append([float(v) for v in y])
        hs.append([float(v) for v in h])
        invs.append(float(inv))
        if g is not None:
            grow = []
            for k in range(d):
                hp = list(h)
                hm = list(h)
                hp[k] += FD_STEP
                hm[k] -= FD_STEP
                grow.append(float((loss_row(hp, w, g[r], eps32) - loss_row(hm, w, g[r], eps32))
                                  / (2 * FD_STEP)))
            dxs.append(grow)
            if w is not None:
                # L is linear in w: dL/dw_k = g_k * h_k * inv (exact, no step needed), but use the
                # same finite-difference route to stay independent of the analytic formula.
                for k in range(d):
                    wp = list(w)
                    wm = list(w)
                    wp[k] = Fraction(w[k]) + Fraction(1, 10**20)
                    wm[k] = Fraction(w[k]) - Fraction(1, 10**20)
                    dw[k] += (loss_row(h, wp, g[r], eps32) - loss_row(h, wm, g[r], eps32)) / (
                        2 * FD_STEP)
    out["expect_y"] = ys
    out["expect_h"] = hs
    out["expect_inv_rms"] = invs
    if g is not None:
        out["expect_dx"] = dxs
        out["expect_dweight"] = [float(v) for v in dw] if dw is not None else None
    return out


def gauss_rows(rng, rows, d, scale=1.0, rounder=f32):
    return [[rounder(rng.gauss(0.0, scale)) for _ in range(d)] for _ in range(rows)]


def main():
    cases = []
    # Reference known answer: Rust RMSNorm test, x=[1,2,3,4], gamma=1, eps=1e-5 -> y0 ~ 0.365148.
    cases.append(make_case("kat_rust_direct", [[1.0, 2.0, 3.0, 4.0]], None, [1.0] * 4,
                           [[1.0] * 4], 1e-5, "tests/core_engine_tests.rs:243-247"))
    cases.append(make_case("kat_rust_split", [[0.5, 1.0, 1.5, 2.0]], [[0.5, 1.0, 1.5, 2.0]],
                           [1.0] * 4, [[1.0] * 4], 1e-5,
                           "same known answer with h = x + residual split in halves"))
    # Reference gradcheck inputs (grad_out = 1, weight = 1, eps = 1e-6 default).
    cases.append(make_case("gradcheck_beast", [[f32(1.2), f32(0.5), f32(-1.0), f32(2.0)]], None,
                           [1.0] * 4, [[1.0] * 4], 1e-6, "tests/test_velograd_beast.py:121"))
    cases.append(make_case("gradcheck_omnibus", [[f32(1.1), f32(-0.5), f32(0.8), f32(1.9)]], None,
                           [1.0] * 4, [[1.0] * 4], 1e-6,
                           "tests/test_velograd_omnibus_grand_master.py:125"))
    rng = random.Random(20260101)
    d = 64
    cases.append(make_case(
        "random_f32_res_w", gauss_rows(rng, 3, d), gauss_rows(rng, 3, d),
        [f32(1.0 + 0.1 * rng.gauss(0, 1)) for _ in range(d)], gauss_rows(rng, 3, d), 1e-5,
        "seeded N(0,1) rows, weight 1+0.1N(0,1)"))
    d = 48
    cases.append(make_case("random_f32_plain", gauss_rows(rng, 2, d), None, None,
                           gauss_rows(rng, 2, d), 1e-6, "no residual, no weight"))
    d = 40
    cases.append(make_case(
        "random_bf16_res_w", gauss_rows(rng, 4, d, rounder=bf16),
        gauss_rows(rng, 4, d, rounder=bf16),
        [bf16(1.0 + 0.1 * rng.gauss(0, 1)) for _ in range(d)],
        gauss_rows(rng, 4, d, rounder=bf16), 1e-5, "bfloat16-representable inputs"))
    d = 32
    zero = [0.0] * d
    const = [0.75] * d
    outl = [f32(rng.gauss(0, 2.0)) for _ in range(d)]
    outl[5] = f32(outl[5] * 50.0)
    cases.append(make_case(
        "special_rows", [zero, const, outl], None,
        [f32(1.0 + 0.1 * rng.gauss(0, 1)) for _ in range(d)], gauss_rows(rng, 3, d), 1e-6,
        "zero row (inv_rms = eps^-1/2, y = 0), constant row, one x50 outlier"))
    with open(OUT, "w") as f:
        json.dump({"generator": "tests/golden/make_golden.py", "cases": cases}, f, indent=0)
    print(f"wrote {OUT}: {len(cases)} cases")


if __name__ == "__main__":
    main()
