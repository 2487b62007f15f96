"""Writes tests/golden/field_env.json from the reference core's env protocol
(the compiled csim of oracle/_ref through oracle/ref_driver.c, the reference
CPU env's reset / step, complete_port/pufferlib_cpu_env.h:187-257) on
FDM-scale env scenarios (generate.field_env_writer: an FDM plan's field with
one VAV per room), run only here, in the development container:

    python tests/golden/make_field_env.py

Per case: the scenario spec (the generator regenerates the blob; its SHA-256
is recorded so a generator change is caught), the env (occupancy seed, start,
max_steps), the action seed, and per step the float32 reward bits and the
SHA-256 of the observation prefix and of the full state snapshot (field,
interior mass, HVAC state; ref_state's order), plus a few values for readable
failures. Action rows are pyoracle.action_row(ACTION_SEED, env, step).
"""
from __future__ import annotations

import hashlib
import json
import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))

from neurips2026_smart_building_challenge_amd.scenario import fdm as F  # noqa: E402
from neurips2026_smart_building_challenge_amd.scenario import generate as G  # noqa: E402

OUT = Path(__file__).resolve().parent / "field_env.json"
ACTION_SEED = 20261202
TABLE_STEPS = G.EPISODE_STEPS + 256
# name, field spec, AHUs, climate index, occ_seed, env index (action rows), start, max_steps, steps,
# stochastic convection (p, distance, seed) or None. The cases at start 0 use the
# blob's occupancy seed (17321), as the first env of a vec on the blob does (its
# convection stream then has the blob's conv_seed). The convection cases use the
# shipped buildings' setting, p = 0.1 within distance 2 (data/blob_meta/*.json).
SHIPPED_CONV = (0.1, 2, 5)
CASES = [
    ("field_small", dict(rows=120, cols=90, rooms=7, margin=6, seed=3), 2, 1, 17321, 0, 0, 40, 60, None),
    ("field_small_offset", dict(rows=120, cols=90, rooms=7, margin=6, seed=3), 2, 1, 78, 1, 200, 30, 45, None),
    ("field_train1_size", dict(), 3, 3, 17321, 0, 0, 8640, 3, None),
    ("field_small_conv", dict(rows=120, cols=90, rooms=7, margin=6, seed=3), 2, 1, 17321, 0, 0, 30, 45,
     SHIPPED_CONV),
    ("field_train1_conv", dict(), 3, 3, 17321, 0, 0, 8640, 4, SHIPPED_CONV),
]


def spec_of(field: dict, ahus: int) -> G.FieldEnvSpec:
    return G.FieldEnvSpec(F.FdmSpec(**field), ahus)


def blob(field: dict, ahus: int, clim: int, tmp: Path, conv=None) -> tuple[Path, str]:
    spec = spec_of(field, ahus)
    cv = None if conv is None else G.ConvSpec(*conv)
    data = G.field_env_writer(spec, G.climates()[clim], TABLE_STEPS, 17321, cv).tobytes()
    p = tmp / f"{spec.name}__c{clim}{'' if cv is None else '__' + cv.tag}.sbb"
    p.write_bytes(data)
    return p, hashlib.sha256(data).hexdigest()


def digest(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def run_case(kind: str, path: Path, occ_seed: int, env: int, start: int, max_steps: int, steps: int) -> dict:
    import pyoracle as po

    e = po.CpuEnv(kind, path, occ_seed, start=start, max_steps=max_steps)
    n = e.obs_len
    ob = e.reset()
    rec = {"obs_sha": [digest(ob[:n])], "state_sha": [digest(e.state())], "reward_bits": [], "terminal": [],
           "obs_head": [ob[:8].tolist()]}
    for s in range(steps):
        row = po.action_row(ACTION_SEED, env, s, e.n_cont, e.n_disc)
        ob, r, t, _ = e.step(row)
        st = e.state()
        rec["obs_sha"].append(digest(ob[:n]))
        rec["state_sha"].append(digest(st))
        rec["reward_bits"].append(int(np.float32(r).view(np.uint32)))
        rec["terminal"].append(float(t))
        rec["obs_head"].append(ob[:8].tolist())
    e.close()
    return rec


def main() -> None:
    import pyoracle as po

    if not po.ref_available():
        raise SystemExit("oracle/_ref is not built (needs /root/reference)")
    out = {"action_seed": ACTION_SEED, "table_steps": TABLE_STEPS, "cases": {}}
    with tempfile.TemporaryDirectory() as td:
        for name, field, ahus, clim, occ, env, start, ms, steps, conv in CASES:
            path, sha = blob(field, ahus, clim, Path(td), conv)
            rec = run_case("ref", path, occ, env, start, ms, steps)
            rec.update({"field": field, "ahus": ahus, "climate": clim, "occ_seed": occ, "env": env, "start": start,
                        "max_steps": ms, "steps": steps, "blob_sha256": sha, "conv": conv})
            out["cases"][name] = rec
            print(name, "ok", flush=True)
    OUT.write_text(json.dumps(out, indent=1))


if __name__ == "__main__":
    main()
