"""Host-side sampler arithmetic and the golden step transitions of the
reference's Euler sampler (tests/golden/sampler_update_ref.npz, made by
tests/golden/make_sampler_golden.py from the reference build)."""
import numpy as np

COMBOS = ("t", "s", "c", "ts", "tc", "sc", "tsc")


def euler_times(step, steps, init_scale):
    """sampler.c:243-246: (timestep, dt = timestep_next - timestep), float32."""
    f = np.float32
    u = f(step) / f(steps)
    un = f(step + 1) / f(steps)
    t = f(f(1.0) - u) * f(init_scale)
    tn = f(f(1.0) - un) * f(init_scale)
    return f(t), f(tn - t)


def cfg_rows(scales):
    """sampler.c:133-139: unconditional rows of the text, speaker and caption
    branches (-1 without CFG), given every branch has context tokens."""
    text, speaker, caption = (int(s > 0) for s in scales)
    return (1 if text else -1, 1 + text if speaker else -1, 1 + text + speaker if caption else -1)


def transitions(Z, flavour, name):
    """Yield (state, velocity rows, use_cfg, rows, scales, dt, next_state,
    traced timestep, timestep) for every step of one trace."""
    cfg = Z[f"{flavour}_{name}_cfg"]
    steps, init = int(cfg[0]), float(cfg[1])
    scales, cfg_min, cfg_max = cfg[2:5], cfg[5], cfg[6]
    states = Z[f"{flavour}_{name}_states"]
    vel = Z[f"{flavour}_{name}_velocity"]
    batch = Z[f"{flavour}_{name}_batch"]
    traced = Z[f"{flavour}_{name}_timestep"]
    rows = cfg_rows(scales)
    max_batch = 1 + sum(r >= 0 for r in rows)
    for s in range(steps):
        t, dt = euler_times(s, steps, init)
        use_cfg = max_batch > 1 and cfg_min <= t <= cfg_max  # sampler.c:247-249
        assert int(batch[s]) == (max_batch if use_cfg else 1)
        yield (states[s], vel[s][: int(batch[s])], use_cfg, rows, scales, dt, states[s + 1],
               traced[s], t)
