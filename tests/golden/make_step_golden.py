"""Write tests/golden/dit_step_ref.npz: the DiT evaluation of one sampler
step (sampler.c:259-278) of the reference's scalar build over two layers
with distinct seeded weights: iro_dit_input on one latent row set, broadcast
to the CFG rows, iro_dit_block_shared_context per layer (int8 weights, the
default two-term W2), iro_dit_output.  The reference is compiled from its
sources by `make -C oracle ref` (oracle/_ref/libref_strict.so).  The fixture
stores the velocity, the velocity of the same evaluation at batch 1 (a
plain step, sampler.c:247-249, which reads row 0 of the CFG mask) and a
SHA-256 digest of the seeded inputs that step_inputs() regenerates bit for
bit.  Re-run after changing the case:

    python tests/golden/make_step_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
sys.path.insert(0, os.path.join(REPO, "irodori-c_amd"))

from iro_synth import gauss  # noqa: E402

D, H, R, LAT = 1280, 3680, 192, 32  # MODEL_DIM, MLP_DIM, ADALN_RANK, LATENT_DIM (dit.c:12-20)
B, S, C, LAYERS = 3, 20, 12, 2
EPS = 1e-6


def step_inputs():
    """x [S, 32], cond [B, 3D] (the same row for every CFG row, as the sampler
    broadcasts it), head (in_w, in_b, out_norm, out_w, out_b), per layer 18
    adaLN arrays and 10 block arrays, the shared context rows [C, D] and the
    CFG mask [B, C]."""
    x = gauss(800, (S, LAT))
    cond = np.repeat(gauss(801, (1, 3 * D), 0.5), B, axis=0)
    head = [gauss(802, (D, LAT), 0.2), gauss(803, (D,), 0.1), gauss(804, (D,), 0.2) + 1.0,
            gauss(805, (LAT, D), 0.03), gauss(806, (LAT,), 0.1)]
    ada, blk = [], []
    for l in range(LAYERS):
        base = 900 + 100 * l
        for i in range(6):
            ada += [gauss(base + 3 * i, (R, D), 0.05), gauss(base + 3 * i + 1, (D, R), 0.05),
                    gauss(base + 3 * i + 2, (D,), 0.1)]
        blk += [gauss(base + 20 + i, (D, D), 0.03) for i in range(5)]
        blk += [gauss(base + 25, (D,), 0.2) + 1.0, gauss(base + 26, (D,), 0.2) + 1.0]
        blk += [gauss(base + 27, (H, D), 0.03), gauss(base + 28, (H, D), 0.03),
                gauss(base + 29, (D, H), 0.02)]
    ck, cv = gauss(807, (C, D)), gauss(808, (C, D))
    mask = np.ones((B, C), np.uint8)
    mask[1, :5] = 0   # a text-unconditional row
    mask[2, 5:] = 0   # a speaker-unconditional row
    return x, cond, head, ada, blk, ck, cv, mask


def input_digest(x, cond, head, ada, blk, ck, cv):
    h = hashlib.sha256()
    for a in [x, cond, *head, *ada, *blk, ck, cv]:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def main():
    from oracle import Reference
    x, cond, head, ada, blk, ck, cv, mask = step_inputs()
    ref = Reference("strict")
    vel = ref.dit_step(x, cond, head, ada, blk, ck, cv, mask, B, S, EPS)
    vel1 = ref.dit_step(x, cond[:1], head, ada, blk, ck, cv, mask[:1], 1, S, EPS)
    path = os.path.join(HERE, "dit_step_ref.npz")
    inputs = input_digest(x, cond, head, ada, blk, ck, cv)
    np.savez_compressed(path, velocity=vel, velocity_b1=vel1, mask=mask,
                        inputs_sha256=np.array(inputs))
    print(f"wrote {path}: velocity {vel.shape}, inputs {inputs[:16]}")


if __name__ == "__main__":
    main()
