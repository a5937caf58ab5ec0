"""Write tests/golden/dit_block_ref.npz: one DiT block of the reference's
scalar build (iro_dit_block, dit.c:1042-1047, layer 0) on seeded inputs.

The reference is compiled from its sources by `make -C oracle ref`
(oracle/_ref/libref_strict.so, the -O2 build of the reference Makefile).
The adaLN low-rank weights are zero, so each adaLN branch is its bias plus
its slice of cond and the gates are glibc's tanhf of that (dit.c:543-588);
the fixture stores those six parameter rows per batch (what the device block
takes as input), the block's output x, and SHA-256 digests of the seeded
inputs that block_inputs() regenerates bit for bit.  Re-run after changing
the case:

    python tests/golden/make_block_golden.py
"""
import ctypes
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
sys.path.insert(0, os.path.join(REPO, "irodori-c_amd"))

from iro_synth import gauss  # noqa: E402

D, H = 1280, 3680       # MODEL_DIM, MLP_DIM of dit.c:12-20
B, S, C = 2, 24, 9
EPS = 1e-6


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def block_inputs():
    """x, cond, the six adaLN biases, the block's fp32 weights (wq, wk, wv,
    wgate, wo, q_norm, k_norm, w1, w3, w2), context rows and mask."""
    x = gauss(700, (B * S, D))
    cond = gauss(701, (B, 3 * D), 0.5)
    ada = gauss(702, (6, D), 0.1)
    w = [gauss(703 + i, (D, D), 0.03) for i in range(5)]
    w += [gauss(708, (D,), 0.2) + 1.0, gauss(709, (D,), 0.2) + 1.0]
    w += [gauss(710, (H, D), 0.03), gauss(711, (H, D), 0.03), gauss(712, (D, H), 0.02)]
    ck, cv = gauss(713, (B * C, D)), gauss(714, (B * C, D))
    mask = np.zeros((B, C), np.uint8)
    mask[0, [0, 1, 4, 8]] = 1
    mask[1, :] = 1
    return x, cond, ada, w, ck, cv, mask


def ada_params(cond, ada):
    """[2, 3, B, D]: (shift, scale, tanhf(gate)) of the attention and MLP
    adaLN with zero low-rank weights: bias + cond slice, rounded once."""
    libm = ctypes.CDLL("libm.so.6")
    libm.tanhf.restype = ctypes.c_float
    libm.tanhf.argtypes = [ctypes.c_float]
    out = np.empty((2, 3, B, D), np.float32)
    for half in range(2):
        for br in range(3):
            v = (ada[3 * half + br][None, :] + cond[:, br * D:(br + 1) * D]).astype(np.float32)
            if br == 2:
                v = np.array([[libm.tanhf(float(t)) for t in row] for row in v], np.float32)
            out[half, br] = v
    return out


def main():
    from oracle import Reference
    x, cond, ada, w, ck, cv, mask = block_inputs()
    ref = Reference("strict")
    y = ref.dit_block_zero_adaln(x, cond, ada, w, ck, cv, mask, B, S, EPS, use_int8=True)
    params = ada_params(cond, ada)
    inputs = digest(np.concatenate([a.ravel() for a in [x, cond, ada, *w, ck, cv]]))
    path = os.path.join(HERE, "dit_block_ref.npz")
    np.savez_compressed(path, x_out=y, ada=params, mask=mask, inputs_sha256=np.array(inputs))
    print(f"wrote {path}: x_out {y.shape}, inputs {inputs[:16]}")


if __name__ == "__main__":
    main()
