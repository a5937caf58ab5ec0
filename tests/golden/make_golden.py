"""Write tests/golden/int8_ref_vectors.npz from the reference's own int8 path.

Runs the reference's ops.c / dacvae.c as compiled from its sources by
`make -C oracle ref` (oracle/_ref/libref_{strict,fast}.so, the -O2 and the
-O3 -march=native -ffast-math builds of the reference Makefile) on small
seeded inputs and stores inputs and outputs, plus SHA-256 digests of the
outputs at the BASELINE shapes (whose inputs iro_synth regenerates bit for
bit from their seeds).  Re-run after changing the cases:

    python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
sys.path.insert(0, os.path.join(REPO, "irodori-c_amd"))

from iro_synth import gauss, heavy_tail, rms_rows  # noqa: E402
from oracle import Oracle, Reference  # noqa: E402


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def small_inputs():
    x = gauss(501, (9, 96))
    x[1] = 0.0
    x[2] = 2.5
    x[3, 17] = 20.0
    w = gauss(502, (40, 96), 0.02)
    w[3] = 0.0
    b = gauss(503, (40,), 0.01)
    y0 = gauss(504, (9, 40))
    cx = gauss(505, (50, 16))
    cx[10:30] = 0.0
    cw = gauss(506, (24, 7 * 16), 0.02)
    cb = gauss(507, (24,), 0.01)
    sa = gauss(508, (4096,), 4.0)
    sg = gauss(509, (4096,))
    return dict(x=x, w=w, b=b, y0=y0, cx=cx, cw=cw, cb=cb, sa=sa, sg=sg)


def baseline_inputs():
    """cfg0 single linear and the QKVG input rows (seeds fixed here)."""
    x0 = gauss(601, (256, 1024))
    w0 = gauss(602, (1024, 1024), 0.02)
    b0 = gauss(603, (1024,), 0.01)
    x1 = heavy_tail(rms_rows(gauss(604, (2250, 1024))), 605)
    return x0, w0, b0, x1


def main():
    out = {}
    inp = small_inputs()
    out.update({f"in_{k}": v for k, v in inp.items()})
    o = Oracle()
    x0, w0, b0, x1 = baseline_inputs()
    for flavour in ("strict", "fast"):
        r = Reference(flavour)
        p = flavour + "_"
        wq = r.weight_quantize(inp["w"])
        out[p + "wq"], out[p + "ws"], out[p + "wcs"] = wq
        q = r.quantize_rows(inp["x"])
        out[p + "q"], out[p + "s"], out[p + "z"] = q
        (q1, s1, z1), res, (q2, s2, z2) = r.quantize_rows_residual(inp["x"])
        for k, v in dict(q1=q1, s1=s1, z1=z1, res=res, q2=q2, s2=s2, z2=z2).items():
            out[p + "r_" + k] = v
        for bias in (0, 1):
            for acc in (0, 1):
                y, work = r.linear(*q, *wq, bias=inp["b"] if bias else None, y=inp["y0"],
                                   accumulate=acc)
                out[f"{p}y_b{bias}_a{acc}"] = y
                out[f"{p}work"] = work
        cwq = r.weight_quantize(inp["cw"])
        out[p + "cwq"], out[p + "cws"], out[p + "cwcs"] = cwq
        for res_ in (0, 1):
            out[f"{p}conv_r{res_}"] = r.conv1d(inp["cx"], *cwq, 7, 1, 3, 9, bias=inp["cb"],
                                               residual=res_, out_len=50)
        out[p + "silu"] = r.silu_mul(inp["sa"], inp["sg"])
        # BASELINE-shape digests
        wq0 = r.weight_quantize(w0)
        q0 = r.quantize_rows(x0)
        y0, work0 = r.linear(*q0, *wq0, bias=b0)
        q1_ = r.quantize_rows(x1)
        out[p + "digests"] = np.array([digest(wq0[0]), digest(wq0[1]), digest(q0[0]),
                                       digest(q0[1]), digest(work0), digest(y0),
                                       digest(q1_[0]), digest(q1_[1]), digest(q1_[2])])
    del o
    path = os.path.join(HERE, "int8_ref_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
