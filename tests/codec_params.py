"""Synthetic DACVAE decoder parameters at the reference's shapes
(dacvae.c:164-221: latent 1024 -> 1536 channels, four upsampling stages of
rates 12, 10, 8, 2 to 768, 384, 192, 96 channels, three residual units of
dilations 1, 3, 9 per stage), random-initialised with a seeded generator."""
from __future__ import annotations

import numpy as np

LATENT, CHANNELS, CODEBOOK, FINAL = 1024, 1536, 32, 96
C_IN = (1536, 768, 384, 192)
C_OUT = (768, 384, 192, 96)
RATES = (12, 10, 8, 2)
DILATIONS = (1, 3, 9)


def _w(rng, shape, fan_in):
    return (rng.standard_normal(shape, dtype=np.float32) / np.float32(np.sqrt(fan_in)))


def _alpha(rng, n):
    return (rng.random(n, dtype=np.float32) * 1.5 + 0.1).astype(np.float32)


def _bias(rng, n):
    return (rng.standard_normal(n, dtype=np.float32) * 0.05).astype(np.float32)


def residual_unit(rng, C, dil):
    return dict(alpha0=_alpha(rng, C), w0=_w(rng, (C, 7, C), 7 * C), b0=_bias(rng, C),
                alpha1=_alpha(rng, C), w1=_w(rng, (C, 1, C), C), b1=_bias(rng, C), dil=dil)


def decoder(seed: int) -> dict:
    """Host arrays in the export layouts of dacvae.h:11-34."""
    rng = np.random.default_rng(seed)
    p = dict(quant_w=_w(rng, (LATENT, 1, CODEBOOK), CODEBOOK), quant_b=_bias(rng, LATENT),
             initial_w=_w(rng, (CHANNELS, 7, LATENT), 7 * LATENT), initial_b=_bias(rng, CHANNELS),
             latent_channels=LATENT, channels=CHANNELS, stages=[])
    for s in range(4):
        r = RATES[s]
        st = dict(alpha=_alpha(rng, C_IN[s]),
                  up_w=_w(rng, (C_IN[s], 2 * r, C_OUT[s]), C_IN[s] * 2),
                  up_b=_bias(rng, C_OUT[s]), c_in=C_IN[s], c_out=C_OUT[s], kernel=2 * r,
                  stride=r, padding=(r + 1) // 2, output_padding=r & 1,
                  residual=[residual_unit(rng, C_OUT[s], d) for d in DILATIONS])
        p["stages"].append(st)
    p["final_alpha"] = _alpha(rng, FINAL)
    p["final_w"] = _w(rng, (1, 7, FINAL), 7 * FINAL)
    p["final_b"] = _bias(rng, 1)
    return p


def reference_order(p: dict) -> list:
    """The 91 arrays in the order the reference driver's decode wrapper reads."""
    out = [p["quant_w"], p["quant_b"], p["initial_w"], p["initial_b"]]
    for st in p["stages"]:
        out += [st["alpha"], st["up_w"], st["up_b"]]
        for u in st["residual"]:
            out += [u["alpha0"], u["w0"], u["b0"], u["alpha1"], u["w1"], u["b1"]]
    out += [p["final_alpha"], p["final_w"], p["final_b"]]
    return out


def to_device(ctx, p: dict) -> dict:
    """The int8-core parameters as device arrays for iro_hip.DACVAE."""
    d = dict(initial_w=ctx.to_device(p["initial_w"]), initial_b=ctx.to_device(p["initial_b"]),
             latent_channels=p["latent_channels"], channels=p["channels"], stages=[])
    for st in p["stages"]:
        e = {k: st[k] for k in ("c_in", "c_out", "kernel", "stride", "padding",
                                "output_padding")}
        e.update(alpha=ctx.to_device(st["alpha"]), up_w=ctx.to_device(st["up_w"]),
                 up_b=ctx.to_device(st["up_b"]), residual=[])
        for u in st["residual"]:
            e["residual"].append({k: (u[k] if k == "dil" else ctx.to_device(u[k])) for k in u})
        d["stages"].append(e)
    return d
