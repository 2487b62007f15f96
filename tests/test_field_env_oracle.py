"""Pins the oracle's env on FDM-scale scenarios (generate.field_env_writer: an
FDM plan's field with one VAV per room) to the reference core:

  - against tests/golden/field_env.json, written by the reference core's own
    env protocol (tests/golden/make_field_env.py): every step's observation
    prefix and full state snapshot (field, interior mass, HVAC state)
    bit-identical (SHA-256), the float32 rewards and terminals equal, on a
    7-room plan (an auto-reset at 40 steps, a calendar offset) and on a plan
    at building_train_1's size (606 x 339 cells, 39 rooms), each also with
    stochastic convection on at the shipped buildings' p = 0.1, distance 2;
  - against the compiled reference core directly (oracle/_ref) where it is
    built;
  - the blob's own structure: every room is a zone with one VAV and one
    area-weighted air-side column, zone areas are the rooms' floor areas; the
    convection candidates are each room's other cells within Chebyshev
    distance 2 (checked cell by cell against a brute-force search).
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import pyoracle as po
from neurips2026_smart_building_challenge_amd.scenario import fdm as F
from neurips2026_smart_building_challenge_amd.scenario import generate as G
from neurips2026_smart_building_challenge_amd.scenario.sbb import read_sbb

GOLDEN = Path(__file__).resolve().parent / "golden"


def fixture() -> dict:
    return json.loads((GOLDEN / "field_env.json").read_text())


def digest(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def write_case(case: dict, table_steps: int, tmp: Path) -> Path:
    spec = G.FieldEnvSpec(F.FdmSpec(**case["field"]), case["ahus"])
    cv = None if case.get("conv") is None else G.ConvSpec(*case["conv"])
    data = G.field_env_writer(spec, G.climates()[case["climate"]], table_steps, 17321, cv).tobytes()
    assert hashlib.sha256(data).hexdigest() == case["blob_sha256"], "stale fixture: the generator changed"
    p = tmp / f"{spec.name}__c{case['climate']}{'' if cv is None else '__' + cv.tag}.sbb"
    p.write_bytes(data)
    return p


def run(kind: str, path: Path, case: dict, seed: int):
    e = po.CpuEnv(kind, path, case["occ_seed"], start=case["start"], max_steps=case["max_steps"])
    n = e.obs_len
    ob = e.reset()
    yield ob[:n], e.state(), None, None
    for s in range(case["steps"]):
        ob, r, t, _ = e.step(po.action_row(seed, case["env"], s, e.n_cont, e.n_disc))
        yield ob[:n], e.state(), r, t


def test_field_env_blob_structure(tmp_path):
    fx = fixture()
    case = fx["cases"]["field_small"]
    path = write_case(case, fx["table_steps"], tmp_path)
    b = read_sbb(path)
    plan = F.make_plan(F.FdmSpec(**case["field"]))
    Z = plan.k
    assert b["zone_area"].size == Z and b["coupled_vav_idx"].size == Z and int(b["sensed_shape"][0]) == Z
    assert np.array_equal(b["phys_room_idx"], np.arange(Z))
    cells = np.array([c.size for c in plan.room_cells], np.float64)
    assert np.allclose(b["zone_area"], cells * plan.spec.cv_m ** 2)
    assert np.array_equal(np.diff(b["room_offsets"]), cells.astype(np.int32))
    # the air side is not the RC kernel's unit same-node coupling
    assert np.any(np.diff(b["applied_indptr"]) > 1)
    assert "solar_gain_coeff" not in b and float(b["conv_p"][0]) == 0.0


def test_field_conv_tables_brute_force(tmp_path):
    """Each convection cell's candidates are its room's other cells within
    Chebyshev distance 2, in row-major order, by brute force over every cell of
    the 7-room plan; every room is a zone's room."""
    fx = fixture()
    case = fx["cases"]["field_small_conv"]
    b = read_sbb(write_case(case, fx["table_steps"], tmp_path))
    assert float(b["conv_p"][0]) == 0.1 and float(b["conv_distance"][0]) == 2.0
    off, cells = b["conv_room_offsets"], b["conv_room_cells"].reshape(-1, 2)
    coff, cidx = b["conv_cand_offsets"], b["conv_cand_idx"]
    assert np.array_equal(off, b["room_offsets"]) and np.array_equal(cells.reshape(-1), b["room_cells"])
    for rm in range(off.size - 1):
        r0, r1 = int(off[rm]), int(off[rm + 1])
        rc = cells[r0:r1]
        for i in range(r0, r1):
            d = np.max(np.abs(rc - cells[i]), axis=1)
            want = [r0 + j for j in np.flatnonzero((d <= 2) & (d > 0))]
            assert list(cidx[coff[i]:coff[i + 1]]) == want, (rm, i)


@pytest.mark.parametrize("name", ["field_small", "field_small_offset", "field_train1_size", "field_small_conv",
                                  "field_train1_conv"])
def test_oracle_matches_reference_fixture(name, tmp_path):
    fx = fixture()
    case = fx["cases"][name]
    path = write_case(case, fx["table_steps"], tmp_path)
    for s, (ob, st, r, t) in enumerate(run("oracle", path, case, fx["action_seed"])):
        assert digest(ob) == case["obs_sha"][s], (name, s, "observation")
        assert digest(st) == case["state_sha"][s], (name, s, "state")
        if s:
            assert int(np.float32(r).view(np.uint32)) == case["reward_bits"][s - 1], (name, s, "reward")
            assert t == case["terminal"][s - 1], (name, s, "terminal")
    assert sum(case["terminal"]) >= (1 if case["steps"] > case["max_steps"] else 0)


@pytest.mark.skipif(not po.ref_available(), reason="oracle/_ref is built only where /root/reference is present")
@pytest.mark.parametrize("name", ["field_small", "field_small_conv"])
def test_oracle_matches_reference_core(name, tmp_path):
    fx = fixture()
    case = dict(fx["cases"][name], steps=90)
    path = write_case(case, fx["table_steps"], tmp_path)
    for s, (a, b) in enumerate(zip(run("oracle", path, case, 5), run("ref", path, case, 5))):
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1]) and a[2] == b[2] and a[3] == b[3], s
