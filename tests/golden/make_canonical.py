"""Writes the golden fixtures of the canonical-layout / residual mode from the
reference's own Python (read from /root/reference, run only here, in the
development container):

    python tests/golden/make_canonical.py

complete_port/submission/residual_policy.py (the submission: canonical
features, comfort guard, residual decode) over complete_port/submission/
pidw_base.py (the starter kit's PIDWaterResetPolicy, vendored there) is driven
through whole episodes of this repo's synthetic buildings. The network is not
used: its output each step is a seeded normal vector, so the residual decode
sees every sign and the clip. The env between the steps is this repo's C
oracle (pinned bit-exactly to the reference csim core), stepped with the
decoded actions.

Per case and step the fixture holds the base controller's proposal
(continuous float32, discrete 0/1), the decoded action (continuous in
[-1, 1], discrete 0/1), the guard's trust per canonical action slot, the
SHA-256 of the canonical observation (983 float32) and, every 20 steps, the
observation itself, and the PID state at the end. The inputs are regenerated
by the test: the blob (seeded generator), the policy outputs (numpy
default_rng(seed + step).normal), the observations (the oracle env).
"""
from __future__ import annotations

import hashlib
import json
import re
import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))
REF_SUBMISSION = Path("/root/reference/complete_port/submission")

from neurips2026_smart_building_challenge_amd.scenario import generate as G  # noqa: E402
from neurips2026_smart_building_challenge_amd.scenario.sbb import read_sbb  # noqa: E402

OUT = Path(__file__).resolve().parent
CN_OBS, CN_ACT = 983, 219
# name, layout (zones, AHUs), climate, start offset, steps, guard (d0, d1, hot) or None
CASES = [
    ("canon_z36_guard", (36, 4), (2.0, 7.0, 611), 0, 320, (0.5, 1.5, 1)),
    ("canon_z81_plain", (81, 9), (-4.0, 6.0, 612), 1440 * 3 + 200, 320, None),
    ("canon_z45_weekend", (45, 5), (24.0, 8.0, 613), 1440 * 4 + 180, 320, (1.0, 2.0, 0)),
]
RES_SCALE, RES_DSCALE = 0.5, 1.5


def policy_seed(name: str) -> int:
    return int(hashlib.sha256(name.encode()).hexdigest()[:8], 16)


def policy_output(name: str, step: int) -> np.ndarray:
    return np.random.default_rng(policy_seed(name) + step).normal(0.0, 1.2, CN_ACT).astype(np.float32)


def blob_for(layout, climate, tmpdir: Path) -> tuple[Path, str]:
    spec = G.LayoutSpec(*layout)
    clim = G.ClimateSpec(climate[0], climate[1], seed=climate[2])
    p = tmpdir / f"{spec.name}__{clim.name}.sbb"
    data = G.scenario_writer(spec, clim, 2 * G.EPISODE_STEPS, 17321, None).tobytes()
    p.write_bytes(data)
    return p, hashlib.sha256(data).hexdigest()


def building_meta(path: Path) -> dict:
    """The starter kit's building_meta_data for one of this repo's blobs."""
    b = read_sbb(path)
    names = bytes(b["field_names"]).decode().split("\n")
    kind, idx, act, disc = b["act_owner_kind"], b["act_owner_index"], b["act_actuator"], b["act_is_discrete"]
    cont_rank = np.cumsum(disc == 0) - 1
    K = int(b["ahu_const"].size // 9)
    temp, press, recirc = [0] * K, [0] * K, [0] * K
    water, water_dp = [], []
    zone_actions: dict[str, dict[str, int]] = {}
    for i in range(kind.size):
        if disc[i]:
            continue
        ci = int(cont_rank[i])
        if kind[i] == 0:
            [temp, press, recirc][int(act[i])][int(idx[i])] = ci
        elif kind[i] == 2:
            (water if act[i] == 0 else water_dp).append(ci)
        else:
            meas = "supply_air_damper_percentage_command" if act[i] == 0 else "reheat_valve_percentage_command"
            zone_actions.setdefault(f"VAV_{int(idx[i]) + 1}", {})[meas] = ci
    vav_ahu = b["vav_ahu_idx"]
    assign = {f"ahu_{k + 1}": [f"room_{v + 1}" for v in range(vav_ahu.size) if vav_ahu[v] == k] for k in range(K)}
    norm: dict[str, dict[str, float]] = {}
    n_dev = int(b["n_dev"][0])
    for i in range(n_dev):
        meas = re.sub(r"^(VAV_\d+_|ahs_ahu_\d+_|hws_)", "", names[i])
        m, v = float(b["f_norm_mean"][i]), float(b["f_norm_var"][i])
        if meas in norm and v > 0.0:   # a zero variance leaves the field unnormalized (its mean unused)
            assert norm[meas]["sample_mean"] == m and norm[meas]["sample_variance"] == v, meas
        norm[meas] = {"sample_mean": m, "sample_variance": v, "sample_std": float(np.sqrt(v))}
    sc = b["sched_scalars"]
    return {
        "comfort_temp_window": (float(sc[2]), float(sc[3])), "eco_temp_window": (float(sc[4]), float(sc[5])),
        "morning_start_hour": int(sc[0]), "evening_start_hour": int(sc[1]),
        "n_discrete_action": int(disc.sum()), "n_continuous_action": int((disc == 0).sum()),
        "temp_indices": temp, "pressure_indices": press + water_dp, "water_indices": water,
        "recirculation_indices": recirc, "zone_action_indices": zone_actions,
        "observation_field_names": names, "ahu_zone_assignments": assign,
        "observation_normalization_metadata": norm,
    }


def model_dir(tmp: Path, guard) -> Path:
    """A stand-in model directory: zero weights of the smallest network (the
    output is replaced per step), the residual configuration under test."""
    d = tmp / "model"
    d.mkdir(exist_ok=True)
    H, L = 4, 1
    cfg = {"res_scale": RES_SCALE, "res_dscale": RES_DSCALE, "residual": True, "hidden": H, "layers": L,
           "obs_size": CN_OBS, "out_dim": CN_ACT, "weights": "w.bin"}
    if guard:
        cfg.update({"guard_d0": guard[0], "guard_d1": guard[1], "guard_hot": bool(guard[2])})
    (d / "config.json").write_text(json.dumps(cfg))
    np.zeros(H * CN_OBS + (CN_ACT + 1) * H + CN_ACT + L * 3 * H * H, np.float32).tofile(d / "w.bin")
    return d


def run_case(name, layout, climate, start, steps, guard, tmp: Path) -> dict:
    import pyoracle as po

    sys.path.insert(0, str(REF_SUBMISSION))
    import residual_policy as rp

    path, sha = blob_for(layout, climate, tmp)
    meta = building_meta(path)
    pol = rp.ResidualPolicy(meta, None, model_dir=model_dir(tmp, guard))
    assert not pol.fallback
    cap: dict[str, np.ndarray] = {}
    base_get = pol.base.get_action

    def base_cap(o):
        a = base_get(o)
        cap["bc"] = np.asarray(a["continuous_action"], np.float32).copy()
        cap["bd"] = np.asarray(a["discrete_action"], np.int32).copy()
        return a

    feat, trust = pol._features, pol._trust
    pol.base.get_action = base_cap
    pol._features = lambda o, bc, bd: cap.__setitem__("x", feat(o, bc, bd)) or cap["x"]
    pol._trust = lambda o: cap.__setitem__("w", trust(o)) or cap["w"]
    env = po.CpuEnv("oracle", path, 17321, start=start, max_steps=G.EPISODE_STEPS)
    n_obs = env.obs_len
    nC, nD = env.n_cont, env.n_disc
    obs = env.reset()
    rec = {k: [] for k in ("bc", "bd", "cont", "disc", "trust")}
    x_sha = []
    x_full = {}
    for t in range(steps):
        o = obs[:n_obs].astype(np.float32)
        y = policy_output(name, t)
        pol._net = lambda x, y=y: y
        a = pol.get_action(o)
        rec["bc"].append(cap["bc"])
        rec["bd"].append(cap["bd"].astype(np.int8))
        rec["cont"].append(np.asarray(a["continuous_action"], np.float32))
        rec["disc"].append(np.asarray(a["discrete_action"], np.int8))
        rec["trust"].append(cap["w"].astype(np.float32) if "w" in cap else np.ones(CN_ACT, np.float32))
        x = cap["x"][:CN_OBS].astype(np.float32)
        x_sha.append(hashlib.sha256(x.tobytes()).hexdigest())
        if t % 20 == 0:
            x_full[f"x_{t}"] = x
        row = np.zeros(272, np.float32)
        row[:nC] = rec["cont"][-1]
        row[256:256 + nD] = rec["disc"][-1]
        obs, _, _, _ = env.step(row)
    pid = np.array([[pol.base.pid_state[k]["integral"], pol.base.pid_state[k]["prev_error"]]
                    for k in range(len(pol.base.ahu_controllers))])
    env.close()
    np.savez_compressed(OUT / f"{name}.npz", **{k: np.stack(v) for k, v in rec.items()}, pid=pid, **x_full)
    return {"layout": list(layout), "climate": list(climate), "start": start, "steps": steps,
            "guard": list(guard) if guard else None, "res_scale": RES_SCALE, "res_dscale": RES_DSCALE,
            "policy_seed": policy_seed(name), "blob_sha256": sha, "x_sha": x_sha}


def main() -> None:
    if not REF_SUBMISSION.is_dir():
        raise SystemExit("the reference submission code is not here (/root/reference)")
    index = {}
    with tempfile.TemporaryDirectory() as td:
        for name, layout, climate, start, steps, guard in CASES:
            sub = Path(td) / name
            sub.mkdir()
            index[name] = run_case(name, layout, climate, start, steps, guard, sub)
            print(name, "ok", flush=True)
    (OUT / "canonical.json").write_text(json.dumps(index, indent=1))


if __name__ == "__main__":
    main()
