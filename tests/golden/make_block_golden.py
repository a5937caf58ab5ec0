"""Write tests/golden/dit_block_ref.npz: one DiT block of the reference's
scalar build (iro_dit_block, dit.c:1042-1047, layer 0) on seeded inputs.

The reference is compiled from its sources by `make -C oracle ref`
(oracle/_ref/libref_strict.so, the -O2 build of the reference Makefile).
Every weight is seeded, the adaLN low-rank ones included; the fixture stores
the block's output x, the six adaLN parameter rows per batch that the
oracle's restatement of dit.c:543-588 gives (checked against the same
reference build in tests/test_oracle_pins.py), and a SHA-256 digest of the
seeded inputs that block_inputs() regenerates bit for bit.

It also writes tests/golden/dit_block_mask_ref.npz: the same block under the
reference's diagnostic group mask IRO_INT8_MASK (dit.c:273-291, read once
per process, so each mask runs in a child process with the variable set),
for MASKS: all groups fp32, and two mixes that put every group through both
of its paths.  Re-run after changing the case:

    python tests/golden/make_block_golden.py
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

D, H, R = 1280, 3680, 192   # MODEL_DIM, MLP_DIM, ADALN_RANK of dit.c:12-20
MASKS = (0, 5, 10)
B, S, C = 2, 24, 9
EPS = 1e-6


def input_digest(x, cond, ada, w, ck, cv):
    h = hashlib.sha256()
    for a in [x, cond, *ada, *w, ck, cv]:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def block_inputs():
    """x, cond, the 18 adaLN arrays (attention then MLP: down [R, D], up
    [D, R], bias [D] of shift, scale, gate), the block's fp32 weights (wq, wk,
    wv, wgate, wo, q_norm, k_norm, w1, w3, w2), context rows and mask."""
    x = gauss(700, (B * S, D))
    cond = gauss(701, (B, 3 * D), 0.5)
    ada = []
    for i in range(6):
        ada += [gauss(730 + 3 * i, (R, D), 0.05), gauss(731 + 3 * i, (D, R), 0.05),
                gauss(732 + 3 * i, (D,), 0.1)]
    w = [gauss(703 + i, (D, D), 0.03) for i in range(5)]
    w += [gauss(708, (D,), 0.2) + 1.0, gauss(709, (D,), 0.2) + 1.0]
    w += [gauss(710, (H, D), 0.03), gauss(711, (H, D), 0.03), gauss(712, (D, H), 0.02)]
    ck, cv = gauss(713, (B * C, D)), gauss(714, (B * C, D))
    mask = np.zeros((B, C), np.uint8)
    mask[0, [0, 1, 4, 8]] = 1
    mask[1, :] = 1
    return x, cond, ada, w, ck, cv, mask


def block_under_mask(out_path):
    """Child process: the block with the IRO_INT8_MASK of the environment."""
    from oracle import Reference
    x, cond, ada, w, ck, cv, mask = block_inputs()
    y = Reference("strict").dit_block(x, cond, ada, w, ck, cv, mask, B, S, EPS, use_int8=True)
    np.save(out_path, y)


def main():
    import subprocess
    import tempfile
    from oracle import Oracle, Reference
    x, cond, ada, w, ck, cv, mask = block_inputs()
    outs = {}
    with tempfile.TemporaryDirectory() as tmp:
        for m in MASKS:
            path = os.path.join(tmp, f"mask{m}.npy")
            env = dict(os.environ, IRO_INT8_MASK=str(m))
            subprocess.run([sys.executable, os.path.abspath(__file__), "--mask-child", path],
                           env=env, check=True)
            outs[f"x_out_mask{m}"] = np.load(path)
    mpath = os.path.join(HERE, "dit_block_mask_ref.npz")
    np.savez_compressed(mpath, masks=np.array(MASKS), inputs_sha256=np.array(
        input_digest(x, cond, ada, w, ck, cv)), **outs)
    print(f"wrote {mpath}: masks {MASKS}")
    ref = Reference("strict")
    y = ref.dit_block(x, cond, ada, w, ck, cv, mask, B, S, EPS, use_int8=True)
    o = Oracle()
    params = np.stack([o.adaln_params(cond, ada[9 * h:9 * h + 9:3], ada[9 * h + 1:9 * h + 9:3],
                                      ada[9 * h + 2:9 * h + 9:3]) for h in range(2)])
    inputs = input_digest(x, cond, ada, w, ck, cv)
    path = os.path.join(HERE, "dit_block_ref.npz")
    np.savez_compressed(path, x_out=y, ada=params, mask=mask, inputs_sha256=np.array(inputs))
    print(f"wrote {path}: x_out {y.shape}, inputs {inputs[:16]}")


if __name__ == "__main__":
    if len(sys.argv) == 3 and sys.argv[1] == "--mask-child":
        block_under_mask(sys.argv[2])
    else:
        main()
