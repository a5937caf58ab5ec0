"""Write tests/golden/sampler_update_ref.npz: step-by-step traces of the
reference's own Euler sampler (sampler.c, iro_sample_euler_conditions),
built from its sources by `make -C oracle ref` in both flag sets
(oracle/_ref/libref_strict.so, libref_fast.so), on a random-weight DiT
whose weights all alias one seeded pool.  For every CFG combination (text,
speaker and caption unconditional rows, each on or off) the fixture keeps,
per step, the CFG batch, the timestep, the state entering the step and the
velocity rows, plus the sampler's output: each state transition is one
golden vector of the CFG combine + Euler update (sampler.c:281-297).
Steps 0-2 run with CFG (timestep >= cfg_min_t) and step 3 without.
Re-run after changing the cases (about a minute on 8 cores):

    python tests/golden/make_sampler_golden.py
"""
import os
import sys
from concurrent.futures import ProcessPoolExecutor

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
sys.path.insert(0, os.path.join(REPO, "irodori-c_amd"))

from iro_synth import gauss  # noqa: E402

S, STEPS, EPS = 8, 4, 1e-6
# (name, cfg_scale_text, cfg_scale_speaker, cfg_scale_caption)
COMBOS = [("t", 1.5, 0.0, 0.0), ("s", 0.0, 0.75, 0.0), ("c", 0.0, 0.0, 2.25),
          ("ts", 1.5, 0.75, 0.0), ("tc", 1.5, 0.0, 2.25), ("sc", 0.0, 0.75, 2.25),
          ("tsc", 1.5, 0.75, 2.25)]
FLAVOURS = ("strict", "fast")


def case(args):
    flavour, (name, st, ss, sc) = args
    from oracle import Reference
    pool = gauss(1000, (3 * 1280 * 1280,), 0.02)
    text = gauss(1001, (3, 512))
    mask = np.array([1, 0, 1], np.uint8)
    speaker = gauss(1002, (2, 768))
    caption = gauss(1003, (2, 512))
    noise = gauss(1004 + len(name), (S, 32))
    cfg = (STEPS, 1.0, st, ss, sc, 0.3, 1.0)
    out, xt, vel, bt, ts = Reference(flavour).sample_euler(pool, EPS, text, mask, speaker, caption,
                                                           noise, cfg)
    states = np.concatenate([xt[:, 0], out[None]], axis=0)  # [STEPS + 1, S*32]
    return flavour, name, dict(cfg=np.asarray(cfg, np.float32), batch=bt, timestep=ts,
                               states=states, velocity=vel)


def main():
    jobs = [(f, c) for f in FLAVOURS for c in COMBOS]
    arrays = {}
    with ProcessPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        for flavour, name, d in ex.map(case, jobs):
            for k, v in d.items():
                arrays[f"{flavour}_{name}_{k}"] = v
    path = os.path.join(HERE, "sampler_update_ref.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path}: {len(jobs)} traces of {STEPS} steps, {S * 32} latent values per row")


if __name__ == "__main__":
    main()
