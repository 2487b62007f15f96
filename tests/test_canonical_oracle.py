"""Pins the oracle's canonical layout (oracle/sbo_canon.c) against fixtures the
reference's own Python wrote (tests/golden/make_canonical.py: the submission's
residual_policy.py over the starter kit's pid_water base): through whole
episodes of three buildings (4, 5 and 9 air handlers; comfort hours, nights and a
weekend; the comfort guard on and off), the base proposal, the guard's trust, the
canonical observation and the residual decode are bit-identical every step, and the
PID state at the end is equal."""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import pytest

import pyoracle as po
from neurips2026_smart_building_challenge_amd.scenario import generate as G

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))


def _index():
    return json.loads((GOLDEN / "canonical.json").read_text())


def policy_p(seed: int, step: int) -> np.ndarray:
    """The policy's head values of the fixture run (residual_policy.py: p = clip(tanh(y)))."""
    y = np.random.default_rng(seed + step).normal(0.0, 1.2, po.CN_ACT).astype(np.float32)
    return np.clip(np.tanh(y), -1, 1).astype(np.float32)


def canon_blob(case: dict, tmp: Path) -> Path:
    spec = G.LayoutSpec(*case["layout"])
    clim = G.ClimateSpec(case["climate"][0], case["climate"][1], seed=case["climate"][2])
    data = G.scenario_writer(spec, clim, 2 * G.EPISODE_STEPS, 17321, None).tobytes()
    assert hashlib.sha256(data).hexdigest() == case["blob_sha256"], "stale fixture: the generator changed"
    p = tmp / f"{spec.name}__{clim.name}.sbb"
    p.write_bytes(data)
    return p


@pytest.mark.parametrize("name", ["canon_z36_guard", "canon_z81_plain", "canon_z45_weekend"])
def test_canonical_oracle_matches_reference_python(name, tmp_path):
    case = _index()[name]
    fx = np.load(GOLDEN / f"{name}.npz")
    path = canon_blob(case, tmp_path)
    c = po.Canon(path)
    env = po.CpuEnv("oracle", path, 17321, start=case["start"], max_steps=G.EPISODE_STEPS)
    n_obs, nC, nD = env.obs_len, env.n_cont, env.n_disc
    guard = case["guard"]
    obs = env.reset()
    pid = np.zeros(18, np.float64)
    for t in range(case["steps"]):
        o = obs[:n_obs].astype(np.float32)
        base, ai = c.base(o, pid)
        row_base = c.decode(base, np.zeros(po.CN_ACT, np.float32), None, 1, 0.0, 0.0)
        assert np.array_equal(row_base[:nC].view(np.uint32), fx["bc"][t].view(np.uint32)), (name, t, "base")
        assert np.array_equal(row_base[256:256 + nD].astype(np.int8), fx["bd"][t]), (name, t, "base run bits")
        x = c.features(o, base, ai, pid)
        assert hashlib.sha256(x.tobytes()).hexdigest() == case["x_sha"][t], (name, t, "canonical observation")
        if f"x_{t}" in fx:
            assert np.array_equal(x.view(np.uint32), fx[f"x_{t}"].view(np.uint32))
        trust = c.trust(o, guard[0], guard[1], guard[2]) if guard else None
        if guard:
            sl = c.slot_of_action
            assert np.array_equal(trust[sl >= 0].view(np.uint32), fx["trust"][t][sl[sl >= 0]].view(np.uint32)), \
                (name, t, "trust")
        p = policy_p(case["policy_seed"], t)
        row = c.decode(base, p, trust, 1, case["res_scale"], case["res_dscale"])
        assert np.array_equal(row[:nC].view(np.uint32), fx["cont"][t].view(np.uint32)), (name, t, "decode")
        assert np.array_equal(row[256:256 + nD].astype(np.int8), fx["disc"][t]), (name, t, "decode run bits")
        obs, _, _, _ = env.step(row)
    K = c.K
    assert np.array_equal(pid[:2 * K].reshape(K, 2), fx["pid"]), (pid[:2 * K], fx["pid"])
    env.close()
