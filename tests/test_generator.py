"""Synthetic scenario generator: sizes follow the hot-path contract and every
section the reference core reads is present with its dtype."""
from __future__ import annotations

import numpy as np
import pytest

from neurips2026_smart_building_challenge_amd.scenario import generate as G
from neurips2026_smart_building_challenge_amd.scenario.sbb import SbbWriter, read_sbb

# sections csim reads (sb_sim.c:23-98, sb_fdm.c:40-116, sb_occup.c:8-29, sb_convect.c:6-31)
REQUIRED = {
    "grid": np.int64, "solved": np.int64, "capacitance_rate": np.float64, "dirichlet_conductance": np.float64,
    "mass_coupling": np.float64, "mass_retained": np.float64, "mass_gained": np.float64,
    "mass_temp_init": np.float64, "temp_init": np.float64, "horizontal": np.float64, "vertical": np.float64,
    "solver_conductivity": np.float64, "ambient_face_areas_0": np.float64, "ambient_face_areas_1": np.float64,
    "lu_L_indptr": np.int32, "lu_L_indices": np.int32, "lu_L_data": np.float64, "lu_U_indptr": np.int32,
    "lu_U_indices": np.int32, "lu_U_data": np.float64, "lu_perm_r": np.int32, "lu_perm_c": np.int32,
    "applied_indptr": np.int32, "applied_indices": np.int32, "applied_data": np.float64,
    "sensed_indptr": np.int32, "sensed_indices": np.int32, "sensed_data": np.float64, "sensed_shape": np.int64,
    "air_side_sensed_indptr": np.int32, "conv_room_offsets": np.int32, "conv_room_cells": np.int32,
    "conv_cand_offsets": np.int32, "conv_cand_idx": np.int32, "occ_params": np.float64, "occ_hour": np.int64,
    "occ_workday": np.uint8, "zone_area": np.float64, "vav_zone_offsets": np.int32, "room_offsets": np.int32,
    "act_owner_kind": np.uint8, "act_owner_index": np.int32, "act_actuator": np.uint8, "ahu_const": np.float64,
    "vav_const": np.float64, "weather_ambient": np.float64, "sched_comfort": np.float64, "f_dev_kind": np.uint8,
    "f_dev_idx": np.int32, "f_obs_id": np.uint8, "f_norm_mean": np.float64, "f_norm_var": np.float64,
    "aux_time": np.float64, "reward_scalars": np.float64, "rew_hour": np.int64, "rew_month": np.int64,
    "rew_workday": np.uint8, "A_system_data": np.float64, "occ_seed": np.int64,
}


def test_sbb_roundtrip(tmp_path):
    w = SbbWriter()
    w.add("a", np.arange(5), "i64")
    w.add("b", np.ones((2, 3)), "f64")
    w.add("empty", np.zeros(0), "i32")
    w.text("s", "hello")
    w.write(tmp_path / "x.sbb")
    d = read_sbb(tmp_path / "x.sbb")
    assert d["a"].tolist() == [0, 1, 2, 3, 4]
    assert d["b"].shape == (2, 3) and d["empty"].size == 0
    assert bytes(d["s"]) == b"hello"
    raw = (tmp_path / "x.sbb").read_bytes()
    assert raw[:4] == b"SBB1" and len(raw) == int.from_bytes(raw[36:44], "little")


@pytest.mark.parametrize("zones,ahus", G.LAYOUTS)
def test_layout_contract(zones, ahus, tmp_path):
    spec = G.LayoutSpec(zones, ahus)
    p = tmp_path / "s.sbb"
    G.scenario_writer(spec, G.climates()[1], 2 * G.EPISODE_STEPS, 17321).write(p)
    d = read_sbb(p)
    for name, dt in REQUIRED.items():
        assert name in d, name
        assert d[name].dtype == np.dtype(dt), name
    disc = d["act_is_discrete"]
    assert int((disc == 0).sum()) == 2 * zones + 3 * ahus + 2
    assert int((disc == 1).sum()) == ahus + 1
    n_dev, n_aux = int(d["n_dev"][0]), int(d["n_aux"][0])
    assert n_dev == 6 * zones + 10 * ahus + 7 and n_dev + n_aux <= 1024
    assert d["solved"].size == 3 * zones and tuple(d["grid"]) == (3, zones)
    n1 = 2 * G.EPISODE_STEPS + 1
    for name in ("weather_ambient", "sched_comfort", "occ_hour", "rew_hour", "occ_hour_m1", "solar_irradiance"):
        assert d[name].shape[0] == n1, name
    assert d["aux_time"].shape == (n1, n_aux - 1)
    # one VAV per zone, every VAV coupled, AHUs cover contiguous zone blocks
    assert d["coupled_vav_idx"].tolist() == list(range(zones))
    assert sorted(set(d["vav_ahu_idx"].tolist())) == list(range(ahus))


def test_calendar_and_weather():
    cal = G.calendar_tables(2 * 288 * 7 + 1)
    # Monday 00:00 start; weekdays 0..4 are workdays
    assert cal["occ_workday"][:288].all() and not cal["occ_workday"][5 * 288:7 * 288].any()
    assert cal["occ_hour"][12] == 1 and cal["occ_hour_m1"][0] == 23 and cal["occ_workday_m1"][0] == 0
    assert cal["occ_hour_m1"][288] == 23 and cal["occ_workday_m1"][288] == 1
    w = G.weather_tables(G.ClimateSpec(10.0, 8.0, 1), 288 * 30 + 1)
    amb = w["weather_ambient"] - 273.15
    assert abs(amb.mean() - 10.0) < 0.2
    daily = amb[: 288 * 30].reshape(30, 288).mean(0)
    assert daily.argmin() < 12 or daily.argmin() > 276       # coldest around midnight
    assert abs(daily[144] - 18.0) < 0.8                      # warmest at noon, mean + amp
    s = w["solar_irradiance"]
    assert s.max() == pytest.approx(600.0, rel=1e-3) and s[: 6 * 12].max() == 0.0


def test_configs():
    scen, n, offsets = G.config_scenarios(1)
    assert n == 960 and len(scen) == 30 and not offsets
    scen, n, offsets = G.config_scenarios(3)
    assert n == 16384 and offsets
    scen, n, _ = G.config_scenarios(2)
    assert n == 4096 and all(s[0].zones == 81 for s in scen)


def test_convection_tables_are_open_plan_strips():
    """Convection rooms of a synthetic layout: each room is one grid row of one
    floor (its zones' air cells, in column order), every candidate lies in the
    cell's own room within the distance and is not the cell itself, and the
    candidate relation is symmetric (csim draws candidates per cell,
    sb_convect.c:49-55)."""
    for zones, ahus in G.LAYOUTS:
        b, _ = G.layout(G.LayoutSpec(zones, ahus))
        for dist in (1, 2, -1):
            off, cells, coff, cidx = G.conv_tables(b, dist)
            cells = cells.reshape(-1, 2)
            assert off[0] == 0 and off[-1] == cells.shape[0] == zones
            assert np.array_equal(np.sort(cells[:, 1]), np.arange(zones)) and np.all(cells[:, 0] == 0)
            room = np.repeat(np.arange(off.size - 1), np.diff(off))
            pairs = set()
            for c in range(cells.shape[0]):
                fl, r, col = b.zone_pos[cells[c, 1]]
                for k in cidx[coff[c]:coff[c + 1]]:
                    assert k != c and room[k] == room[c]
                    fl2, r2, col2 = b.zone_pos[cells[k, 1]]
                    assert (fl2, r2) == (fl, r)
                    assert dist < 0 or abs(int(col2) - int(col)) <= dist
                    pairs.add((c, int(k)))
            assert all((k, c) in pairs for c, k in pairs)
            for rm in range(off.size - 1):
                cols = [b.zone_pos[z][2] for z in cells[off[rm]:off[rm + 1], 1]]
                assert cols == sorted(cols)
