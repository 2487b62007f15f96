"""Writes the golden fixtures of the env step from the reference csim core.

Run in the development container, where /root/reference exists and
oracle/_ref/libcsim_ref.so has been built from it (oracle/Makefile `ref`):

    python tests/golden/make_golden.py

Every case regenerates its synthetic scenario blob with this repo's seeded
generator, records the blob's SHA-256 (so a generator change is detected as a
stale fixture rather than a parity failure), drives the reference core with the
reference CPU env's reset/step protocol (oracle/ref_driver.c), and stores:

  rewards      f64 per step (the value before the float cast)
  reward_f32   float per step (what the trainer receives)
  obs_*        observation prefix (n_dev + n_aux floats) at recorded steps
  state_*      full state snapshot (ref_state layout) at recorded steps
  sha_obs      SHA-256 over every step's observation prefix
  sha_state    SHA-256 over every step's state snapshot
  total        f64 sum of the episode rewards

Fixtures are small .npz files; the reference itself never leaves this container.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))

from neurips2026_smart_building_challenge_amd.scenario import generate as G  # noqa: E402

OUT = Path(__file__).resolve().parent
ACTION_SEED = 20260501

# name, layout (zones, ahus), climate (mean, amp, seed), occ_seed, start, max_steps, steps, record
# [, convection (p, distance, seed)]
CASES = [
    ("cfg0_episode", (41, 1), (10.0, 8.0, 499), 17321, 0, 8640, 8640,
     [0, 1, 2, 3, 8, 100, 1000, 4320, 8639, 8640]),
    ("z81_autoreset", (81, 4), (28.0, 10.0, 504), 40000, 0, 40, 96, [0, 1, 2, 39, 40, 41, 80, 96]),
    ("z57_offset", (57, 2), (-5.0, 6.0, 500), 31415, 3000, 50, 96, [0, 1, 2, 50, 51, 96]),
    ("z49_weekend", (49, 2), (5.0, 7.0, 501), 2718, 1440, 700, 700, [0, 1, 300, 700]),
    ("z65_convection", (65, 3), (12.0, 8.0, 502), 17321, 0, 40, 96, [0, 1, 2, 40, 41, 96], (0.08, 2, 4321)),
]
# full-episode reward totals (one env per layout, two climates)
TOTALS = [((z, a), (m, amp, 500 + ci)) for (z, a) in G.LAYOUTS for ci, (m, amp) in enumerate(G.CLIMATES)
          if ci in (0, 3)]


def blob_for(layout, climate, tmpdir: Path, conv=None) -> tuple[Path, str]:
    spec = G.LayoutSpec(*layout)
    clim = G.ClimateSpec(climate[0], climate[1], seed=climate[2])
    cv = None if conv is None else G.ConvSpec(*conv)
    p = tmpdir / f"{spec.name}__{clim.name}{'' if cv is None else '__' + cv.tag}.sbb"
    data = G.scenario_writer(spec, clim, 2 * G.EPISODE_STEPS, 17321, cv).tobytes()
    p.write_bytes(data)
    return p, hashlib.sha256(data).hexdigest()


def run_case(kind: str, path: Path, occ_seed: int, start: int, max_steps: int, steps: int, record):
    import pyoracle as po

    env = po.CpuEnv(kind, path, occ_seed, start=start, max_steps=max_steps)
    obs_len = env.obs_len
    h_obs, h_state = hashlib.sha256(), hashlib.sha256()
    rec = {}
    o = env.reset()[:obs_len]
    st = env.state()
    h_obs.update(o.tobytes())
    h_state.update(st.tobytes())
    if 0 in record:
        rec["obs_0"], rec["state_0"] = o, st
    rewards = np.zeros(steps)
    rewards32 = np.zeros(steps, np.float32)
    for s in range(steps):
        row = po.action_row(ACTION_SEED, 0, s, env.n_cont, env.n_disc, kind=kind)
        ob, r, _, _ = env.step(row)
        rewards32[s] = r
        rewards[s] = env.last_reward_f64()
        ob = ob[:obs_len]
        st = env.state()
        h_obs.update(ob.tobytes())
        h_state.update(st.tobytes())
        if s + 1 in record:
            rec[f"obs_{s + 1}"], rec[f"state_{s + 1}"] = ob, st
    env.close()
    return rewards, rewards32, rec, h_obs.hexdigest(), h_state.hexdigest(), obs_len


def main(only: str | None = None) -> None:
    """Writes every fixture, or (only = a case name) that case alone, keeping
    the others and the totals as they are."""
    import pyoracle as po

    if not po.ref_available():
        raise SystemExit("oracle/_ref/libcsim_ref.so is not built (needs /root/reference)")
    tmp = OUT / "_blobs"
    tmp.mkdir(exist_ok=True)
    index = {"action_seed": ACTION_SEED, "cases": {}, "totals": []}
    if only:
        index = json.loads((OUT / "golden.json").read_text())
    for name, layout, climate, occ_seed, start, max_steps, steps, record, *conv in CASES:
        if only and name != only:
            continue
        path, sha = blob_for(layout, climate, tmp, conv[0] if conv else None)
        rewards, r32, rec, ho, hs, obs_len = run_case("ref", path, occ_seed, start, max_steps, steps, record)
        np.savez_compressed(OUT / f"{name}.npz", rewards=rewards, reward_f32=r32, **rec)
        index["cases"][name] = {"layout": list(layout), "climate": list(climate), "occ_seed": occ_seed,
                                "start": start, "max_steps": max_steps, "steps": steps, "record": record,
                                "blob_sha256": sha, "sha_obs": ho, "sha_state": hs, "obs_len": obs_len,
                                "total": float(rewards.sum())}
        if conv:
            index["cases"][name]["conv"] = list(conv[0])
        print(name, "total", rewards.sum())
    for layout, climate in ([] if only else TOTALS):
        path, sha = blob_for(layout, climate, tmp)
        rewards, _, _, ho, hs, _ = run_case("ref", path, 17321, 0, G.EPISODE_STEPS, G.EPISODE_STEPS, [])
        index["totals"].append({"layout": list(layout), "climate": list(climate), "blob_sha256": sha,
                                "total": float(rewards.sum()), "sha_obs": ho, "sha_state": hs})
        print(layout, climate, "total", rewards.sum())
    (OUT / "golden.json").write_text(json.dumps(index, indent=1))
    for p in tmp.glob("*.sbb"):
        p.unlink()
    tmp.rmdir()


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else None)
