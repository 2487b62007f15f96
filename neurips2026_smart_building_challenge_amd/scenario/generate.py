"""Seeded synthetic scenarios (layout x climate) written as SBB1 blobs.

Each blob carries every section the reference core reads (csim/sb_sim.c:23-98,
sb_fdm.c:40-116, sb_occup.c:8-29, sb_convect.c:6-31), with the same names,
dtypes and shapes as the reference baker writes them
(complete_port/pysim/bake_env.py, bake_scenario.py), plus three additions that
csim ignores:

  A_system_{shape,indptr,indices,data}  CSC system matrix (the reference bakes
                                        the same section, bake_scenario.py:125-131)
  solar_irradiance  f64[n1]             W/m^2 per calendar step
  solar_gain_coeff  f64[N]              m^2 per node: q_solar[t] = coeff[t] * I[kk]

Calendar tables hold `table_steps + 1` rows so that an episode of
`episode_steps` may start at any offset in [0, table_steps - episode_steps]
(per-env start offsets, the env kwarg start_offsets). occ_hour_m1 / occ_workday_m1 hold one row per start
offset: the hour/workday of the interval before that start.
"""
from __future__ import annotations

import datetime as _dt
import json
import math
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from .building import AUX_NAMES, DT_SEC, N_AUX, T0, Building, field_name, make_building
from .factor import factorize
from .sbb import SbbWriter

EPISODE_STEPS = 8640
STEPS_PER_DAY = 288
START_DATE = _dt.date(2026, 1, 5)   # a Monday

LAYOUTS = [(41, 1), (49, 2), (57, 2), (65, 3), (73, 3), (81, 4)]
CLIMATES = [(-5.0, 6.0), (5.0, 7.0), (12.0, 8.0), (20.0, 9.0), (28.0, 10.0)]


@dataclass(frozen=True)
class LayoutSpec:
    zones: int
    ahus: int

    @property
    def seed(self) -> int:
        return 1000 + 17 * self.zones + self.ahus

    @property
    def name(self) -> str:
        return f"rc{self.zones:02d}z{self.ahus}a"


@dataclass(frozen=True)
class ClimateSpec:
    mean_c: float
    amp_c: float
    seed: int

    @property
    def name(self) -> str:
        return f"m{self.mean_c:+05.1f}a{self.amp_c:04.1f}".replace("+", "p").replace("-", "n")


COMFORT_HOURS = (6, 19)      # comfort mode on workdays from 06:00 to 19:00
COMFORT_SP = (21.0, 24.0)    # heating / cooling setpoints (C) in comfort mode
ECO_SP = (15.0, 29.0)        # ... and outside it


def calendar_tables(n1: int) -> dict[str, np.ndarray]:
    k = np.arange(n1)
    day = k // STEPS_PER_DAY
    hour = (k % STEPS_PER_DAY) // 12
    frac_hour = (k % STEPS_PER_DAY) / 12.0
    dow = day % 7
    workday = (dow < 5).astype(np.uint8)
    month = np.array([(START_DATE + _dt.timedelta(days=int(d))).month for d in range(int(day[-1]) + 1)])[day]
    h0, h1 = COMFORT_HOURS
    comfort = ((workday == 1) & (hour >= h0) & (hour < h1)).astype(np.float64)
    k_soon = k + 12
    day_s = k_soon // STEPS_PER_DAY
    hour_s = (k_soon % STEPS_PER_DAY) // 12
    comfort_soon = (((day_s % 7) < 5) & (hour_s >= h0) & (hour_s < h1)).astype(np.float64)
    heat = np.where(comfort > 0, T0 + COMFORT_SP[0], T0 + ECO_SP[0])
    cool = np.where(comfort > 0, T0 + COMFORT_SP[1], T0 + ECO_SP[1])
    km1 = k - 1
    day_m1 = np.floor_divide(km1, STEPS_PER_DAY)
    hour_m1 = (km1 % STEPS_PER_DAY) // 12
    workday_m1 = ((day_m1 % 7) < 5).astype(np.uint8)
    aux = np.stack([
        np.cos(2.0 * math.pi * frac_hour / 24.0), np.sin(2.0 * math.pi * frac_hour / 24.0),
        np.cos(2.0 * math.pi * dow / 7.0), np.sin(2.0 * math.pi * dow / 7.0),
        comfort, comfort_soon,
    ], axis=1)
    assert aux.shape[1] == N_AUX - 1
    return {
        "sched_comfort": comfort, "sched_heat_sp": heat, "sched_cool_sp": cool,
        "occ_hour": hour.astype(np.int64), "occ_workday": workday,
        "occ_hour_m1": hour_m1.astype(np.int64), "occ_workday_m1": workday_m1,
        "rew_hour": hour.astype(np.int64), "rew_month": month.astype(np.int64),
        "rew_workday": workday, "aux_time": aux,
    }


def weather_tables(c: ClimateSpec, n1: int) -> dict[str, np.ndarray]:
    """24h sinusoid (minimum at midnight) + N(0,1) noise; half-sine solar, 600 W/m^2 peak."""
    rng = np.random.default_rng(c.seed)
    t = np.arange(n1) * DT_SEC
    amb = T0 + c.mean_c + c.amp_c * np.sin(2.0 * math.pi * t / 86400.0 - math.pi / 2.0) \
        + rng.standard_normal(n1)
    tday = np.mod(t, 86400.0)
    solar = 600.0 * np.maximum(0.0, np.sin(math.pi * (tday - 6 * 3600.0) / (12 * 3600.0)))
    return {"weather_ambient": amb, "solar_irradiance": solar}


def prices() -> dict[str, np.ndarray]:
    per_j = 1.0 / 3.6e6
    wk = np.array([0.10] * 7 + [0.15] * 5 + [0.25] * 6 + [0.15] * 4 + [0.10] * 2) * per_j
    we = np.full(24, 0.09) * per_j
    h = np.arange(24)
    carbon = (0.35 + 0.10 * np.sin(2 * math.pi * (h - 6) / 24.0)) * per_j
    gas = (0.035 - 0.01 * np.cos(2 * math.pi * np.arange(12) / 12.0)) * per_j
    return {"elec_weekday_price": wk, "elec_weekend_price": we,
            "elec_carbon_rate": carbon, "gas_month_price": gas,
            "gas_carbon_rate": 0.181 * per_j}


_LAYOUT_CACHE: dict[tuple[int, int], tuple[Building, dict]] = {}


def layout(spec: LayoutSpec) -> tuple[Building, dict]:
    key = (spec.zones, spec.ahus)
    if key not in _LAYOUT_CACHE:
        b = make_building(spec.zones, spec.ahus, spec.seed, name=spec.name)
        _LAYOUT_CACHE[key] = (b, factorize(b.A))
    return _LAYOUT_CACHE[key]


@dataclass(frozen=True)
class ConvSpec:
    """Stochastic convection (complete_port/csim/sb_convect.c:39-73): each step,
    every cell of a convection room starts a swap with probability p with one of
    its candidates (cells of the same room within `distance` grid columns; -1:
    the whole room); the swaps are shuffled and applied to the field."""
    p: float = 0.05
    distance: int = 2
    seed: int = 9001

    @property
    def tag(self) -> str:
        return f"cv{int(round(self.p * 1000)):03d}d{self.distance}"


def conv_tables(b: Building, distance: int):
    """Convection rooms of a synthetic layout: the zones of one grid row of one
    floor form an open-plan strip, and a strip's room cells are its zones' air
    cells (grid row 0, column z) in column order. Tables in the reference
    baker's form (complete_port/pysim/bake_scenario.py:162-186): room offsets
    into the cell list, cells as (row, col), and per cell a CSR list of its
    candidates as cell positions in that list."""
    rooms: dict[tuple[int, int], list[tuple[int, int]]] = {}
    for z in range(b.n_zones):
        fl, r, c = (int(x) for x in b.zone_pos[z])
        rooms.setdefault((fl, r), []).append((c, z))
    off, cells, cand_off, cand_idx = [0], [], [], []
    for key in sorted(rooms):
        strip = sorted(rooms[key])
        base = len(cells)
        for c, z in strip:
            cells.append((0, z))
        off.append(len(cells))
        for i, (c, _) in enumerate(strip):
            cand_off.append(len(cand_idx))
            for j, (c2, _) in enumerate(strip):
                if j != i and (distance < 0 or abs(c2 - c) <= distance):
                    cand_idx.append(base + j)
    cand_off.append(len(cand_idx))
    return (np.asarray(off, np.int64), np.asarray(cells, np.int64).reshape(-1),
            np.asarray(cand_off, np.int64), np.asarray(cand_idx, np.int64))


def scenario_writer(spec: LayoutSpec, clim: ClimateSpec, table_steps: int,
                    occ_seed: int, conv: ConvSpec | None = None) -> SbbWriter:
    b, f = layout(spec)
    Z, A, N = b.n_zones, b.n_ahu, b.n_nodes
    n1 = table_steps + 1
    w = SbbWriter()
    # ---- grid / field ----
    w.add("grid", [3, Z], "i64")
    w.add("solved", np.arange(N), "i64")
    w.add("capacitance_rate", b.cap_rate, "f64")
    w.add("dirichlet_conductance", b.dirichlet, "f64")
    w.add("mass_coupling", b.mass_coupling, "f64")
    w.add("mass_retained", b.mass_retained, "f64")
    w.add("mass_gained", b.mass_gained, "f64")
    w.add("mass_temp_init", b.mass_temp_init, "f64")
    w.add("temp_init", b.temp_init, "f64")
    w.add("horizontal", np.ones(N), "f64")
    w.add("vertical", np.ones(N), "f64")
    w.add("solver_conductivity", np.ones(N), "f64")
    w.add("ambient_face_areas_0", np.zeros(N), "f64")
    w.add("ambient_face_areas_1", np.zeros(N), "f64")
    w.scalar_f64("convection_coefficient", 8.8)
    Acsc = b.A.tocsc()
    w.add("A_system_shape", [N, N], "i64")
    w.add("A_system_indptr", Acsc.indptr, "i32")
    w.add("A_system_indices", Acsc.indices, "i32")
    w.add("A_system_data", Acsc.data, "f64")
    w.add("lu_perm_r", f["perm_r"], "i32")
    w.add("lu_perm_c", f["perm_c"], "i32")
    w.add("lu_L_shape", [N, N], "i64")
    w.add("lu_L_indptr", f["L_indptr"], "i32")
    w.add("lu_L_indices", f["L_indices"], "i32")
    w.add("lu_L_data", f["L_data"], "f64")
    w.add("lu_U_shape", [N, N], "i64")
    w.add("lu_U_indptr", f["U_indptr"], "i32")
    w.add("lu_U_indices", f["U_indices"], "i32")
    w.add("lu_U_data", f["U_data"], "f64")
    # ---- air side: VAV v supplies and senses the air node of zone v ----
    k = Z
    w.add("applied_shape", [N, k], "i64")
    w.add("applied_indptr", np.arange(k + 1), "i32")
    w.add("applied_indices", np.arange(k), "i32")
    w.add("applied_data", np.ones(k), "f64")
    w.add("sensed_shape", [k, N], "i64")
    w.add("sensed_indptr", np.arange(k + 1), "i32")
    w.add("sensed_indices", np.arange(k), "i32")
    w.add("sensed_data", np.ones(k), "f64")
    ind = np.zeros(N + 1, dtype=np.int64)
    ind[1:Z + 1] = np.arange(1, Z + 1)
    ind[Z + 1:] = Z
    w.add("air_side_sensed_shape", [N, k], "i64")
    w.add("air_side_sensed_indptr", ind, "i32")
    w.add("air_side_sensed_indices", np.arange(k), "i32")
    w.add("air_side_sensed_data", np.ones(k), "f64")
    # ---- convection: off (the BASELINE configs), or on with open-plan strips ----
    if conv is None:
        w.scalar_f64("conv_p", 0.0)
        w.scalar_f64("conv_distance", 0.0)
        w.scalar_i64("conv_seed", 0)
        w.add("conv_room_offsets", [0], "i32")
        w.add("conv_room_cells", np.zeros(0), "i32")
        w.add("conv_cand_offsets", [0], "i32")
        w.add("conv_cand_idx", np.zeros(0), "i32")
    else:
        c_off, c_cells, c_coff, c_idx = conv_tables(b, conv.distance)
        w.scalar_f64("conv_p", conv.p)
        w.scalar_f64("conv_distance", float(conv.distance))
        w.scalar_i64("conv_seed", conv.seed)
        w.add("conv_room_offsets", c_off, "i32")
        w.add("conv_room_cells", c_cells, "i32")
        w.add("conv_cand_offsets", c_coff, "i32")
        w.add("conv_cand_idx", c_idx, "i32")
    # ---- zones / rooms / VAVs: zone z is the air cell of column z ----
    rooms = (np.arange(Z + 1), np.stack([np.zeros(Z, dtype=np.int64), np.arange(Z)], 1).reshape(-1))
    hvac_sections(w, b, Z, clim, table_steps, occ_seed, b.zone_area, b.cv_size_cm, rooms, b.solar_coeff)
    return w


def hvac_sections(w: SbbWriter, b: Building, Z: int, clim: ClimateSpec, table_steps: int, occ_seed: int,
                  zone_area: np.ndarray, cv_size_cm: float, rooms, solar_coeff) -> None:
    """The sections past the field: zones (one VAV per zone, zone z in room
    z), the rooms' cells when `rooms` = (offsets, cells) is given, the HVAC
    plant of `b`, actions, observation, calendar and weather (with the solar
    gain coefficients when given), occupancy and reward tables."""
    n1 = table_steps + 1
    w.add("zone_area", zone_area, "f64")
    w.add("phys_room_idx", np.arange(Z), "i32")
    if rooms is not None:
        w.add("room_offsets", rooms[0], "i32")
        w.add("room_cells", rooms[1], "i32")
    w.add("vav_zone_offsets", np.arange(Z + 1), "i32")
    w.add("vav_zone_idx", np.arange(Z), "i32")
    w.add("zone_vav_offsets", np.arange(Z + 1), "i32")
    w.add("zone_vav_idx", np.arange(Z), "i32")
    w.add("vav_ahu_idx", b.vav_ahu, "i32")
    w.add("coupled_vav_idx", np.arange(Z), "i32")
    w.add("ahu_const", b.ahu_const, "f64")
    w.add("vav_const", b.vav_const, "f64")
    w.scalar_f64("hws_header_resistance", b.header_res)
    w.scalar_f64("hws_is_boiler", 1.0)
    w.add("boiler_const", b.boiler_const, "f64")
    w.add("pump_const", b.pump_const, "f64")
    w.scalar_f64("internal_gain_w_per_m2", b.internal_w_m2)
    w.scalar_f64("internal_gain_standby_fraction", b.standby_frac)
    w.scalar_f64("occupant_sensible_heat_w", b.occupant_w)
    w.scalar_f64("cv_size_cm", cv_size_cm)
    # ---- actions ----
    w.add("act_owner_kind", b.act_kind, "u8")
    w.add("act_owner_index", b.act_index, "i32")
    w.add("act_actuator", b.act_actuator, "u8")
    w.add("act_is_discrete", b.act_is_disc, "u8")
    w.add("act_min_native", b.act_min_native, "f64")
    w.add("act_max_native", b.act_max_native, "f64")
    w.add("act_min_norm", np.full(b.act_kind.size, -1.0), "f64")
    w.add("act_max_norm", np.full(b.act_kind.size, 1.0), "f64")
    # ---- observation ----
    w.add("f_dev_kind", b.f_dev_kind, "u8")
    w.add("f_dev_idx", b.f_dev_idx, "i32")
    w.add("f_obs_id", b.f_obs_id, "u8")
    w.add("f_norm_mean", b.f_norm_mean, "f64")
    w.add("f_norm_var", b.f_norm_var, "f64")
    w.scalar_i64("n_dev", b.f_dev_kind.size)
    w.scalar_i64("n_aux", N_AUX)
    names = [field_name(int(k), int(i), int(o)) for k, i, o in zip(b.f_dev_kind, b.f_dev_idx, b.f_obs_id)]
    w.text("field_names", "\n".join(names + AUX_NAMES))
    # schedule (bake_env.py:103-108): morning / evening start hour, comfort and
    # eco (heating, cooling) windows, as calendar_tables draws them
    w.add("sched_scalars", [float(COMFORT_HOURS[0]), float(COMFORT_HOURS[1]), T0 + COMFORT_SP[0], T0 + COMFORT_SP[1],
                            T0 + ECO_SP[0], T0 + ECO_SP[1]], "f64")
    w.add("obs_meta", [1.0, 1.0, 1.0, float(EPISODE_STEPS), DT_SEC], "f64")
    # ---- calendar / weather / occupancy ----
    cal = calendar_tables(n1)
    wt = weather_tables(clim, n1)
    w.add("weather_ambient", wt["weather_ambient"], "f64")
    w.add("solar_irradiance", wt["solar_irradiance"], "f64")
    if solar_coeff is not None:
        w.add("solar_gain_coeff", solar_coeff, "f64")
    for name in ("sched_comfort", "sched_heat_sp", "sched_cool_sp"):
        w.add(name, cal[name], "f64")
    w.add("occ_hour", cal["occ_hour"], "i64")
    w.add("occ_workday", cal["occ_workday"], "u8")
    w.add("occ_hour_m1", cal["occ_hour_m1"], "i64")
    w.add("occ_workday_m1", cal["occ_workday_m1"], "u8")
    w.add("rew_hour", cal["rew_hour"], "i64")
    w.add("rew_month", cal["rew_month"], "i64")
    w.add("rew_workday", cal["rew_workday"], "u8")
    w.add("aux_time", cal["aux_time"], "f64")
    w.add("occ_params", [2.0, 7.0, 9.0, 17.0, 19.0, DT_SEC], "f64")
    w.scalar_i64("occ_seed", occ_seed)
    # ---- reward ----
    w.add("reward_scalars", [30.0, 10.0, 2.0, 1500.0 * Z, 10000.0 * Z, 0.5, 0.25, 0.25], "f64")
    p = prices()
    for name in ("elec_weekday_price", "elec_weekend_price", "elec_carbon_rate", "gas_month_price"):
        w.add(name, p[name], "f64")
    w.scalar_f64("gas_carbon_rate", p["gas_carbon_rate"])
    w.scalar_i64("table_steps", table_steps)


# ---------------------------------------------------------------- configs ----

def climates() -> list[ClimateSpec]:
    return [ClimateSpec(m, a, seed=500 + i) for i, (m, a) in enumerate(CLIMATES)]


def config_scenarios(config: int) -> tuple[list[tuple[LayoutSpec, ClimateSpec]], int, bool]:
    """(scenarios, n_envs, start_offsets) for the BASELINE configs 0..4 (0-based);
    start_offsets: every env starts at its own seeded calendar offset (config 3,
    BASELINE's "desync on")."""
    lays = [LayoutSpec(z, a) for z, a in LAYOUTS]
    if config == 0:
        return [(LayoutSpec(41, 1), ClimateSpec(10.0, 8.0, seed=499))], 1, False
    mixed = [(l, c) for l in lays for c in climates()]
    if config in (1, 4):
        return mixed, 960, False
    if config == 2:
        return [(LayoutSpec(81, 4), c) for c in climates()], 4096, False
    if config == 3:
        return mixed, 16384, True
    raise ValueError(f"unknown config {config}")


def write_scenarios(scen: list[tuple[LayoutSpec, ClimateSpec]], out_dir,
                    table_steps: int = 2 * EPISODE_STEPS, occ_seed_base: int = 17321,
                    conv: ConvSpec | None = None) -> list[Path]:
    """Writes one blob per scenario; with `conv`, every blob has stochastic
    convection on (scenario i gets conv seed conv.seed + 7 i)."""
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    paths = []
    for i, (l, c) in enumerate(scen):
        cv = None if conv is None else ConvSpec(conv.p, conv.distance, conv.seed + 7 * i)
        tag = "" if conv is None else "__" + conv.tag
        p = out / f"{l.name}__{c.name}{tag}.sbb"
        if not p.exists():
            scenario_writer(l, c, table_steps, occ_seed_base + 101 * i, cv).write(p)
        paths.append(p)
    meta = {"scenarios": [p.name for p in paths], "table_steps": table_steps,
            "episode_steps": EPISODE_STEPS}
    (out / "manifest.json").write_text(json.dumps(meta, indent=1))
    return paths


def write_config(config: int, out_dir, conv: ConvSpec | None = None) -> tuple[list[Path], int, bool]:
    scen, n, offsets = config_scenarios(config)
    return write_scenarios(scen, out_dir, conv=conv), n, offsets


# ------------------------------------------------------ FDM-scale buildings --

@dataclass(frozen=True)
class FieldEnvSpec:
    """A building whose field is an FDM plan (scenario/fdm.py) and whose HVAC
    plant serves one VAV per room: the zones are the plan's rooms, the plant
    constants those of a seeded RC layout with as many zones and `ahus` AHUs."""
    field: "object"           # fdm.FdmSpec
    ahus: int = 3

    @property
    def seed(self) -> int:
        return 5000 + 31 * self.field.rooms + self.ahus + 7 * self.field.seed

    @property
    def name(self) -> str:
        return f"{self.field.name}_a{self.ahus}"


def field_conv_tables(plan, distance: int):
    """Convection rooms of an FDM plan: every room, its cells in row-major
    order, and per cell its candidates, the room's other cells within
    Chebyshev distance `distance` in row-major order (the reference baker's
    table form, complete_port/pysim/bake_scenario.py:162-186: room offsets
    into the cell list, cells as (row, col), candidates as CSR over cell
    positions in that list)."""
    cols = plan.spec.cols
    off, cells, cand_off, cand_idx = [0], [], [np.zeros(1, np.int64)], []
    for rc in plan.room_cells:
        p = plan.solved[rc]
        r, c = p // cols, p % cols
        r0, c0 = int(r.min()), int(c.min())
        h, w = int(r.max()) - r0 + 1, int(c.max()) - c0 + 1
        if h * w != rc.size:
            raise ValueError("convection rooms must be rectangles of the plan")
        base = off[-1]
        cells.append(np.stack([r, c], 1))
        off.append(base + rc.size)
        lr, lc = (r - r0)[:, None], (c - c0)[:, None]
        offs = [(dr, dc) for dr in range(-distance, distance + 1) for dc in range(-distance, distance + 1)
                if (dr, dc) != (0, 0)]
        dr = np.array([o[0] for o in offs])[None, :]
        dc = np.array([o[1] for o in offs])[None, :]
        nr, nc = lr + dr, lc + dc
        ok = (nr >= 0) & (nr < h) & (nc >= 0) & (nc < w)
        cand = np.where(ok, base + nr * w + nc, -1)
        cnt = ok.sum(1)
        cand_idx.append(cand[ok])
        cand_off.append(cand_off[-1][-1] + np.cumsum(cnt))
    return (np.asarray(off, np.int64), np.concatenate(cells).reshape(-1).astype(np.int64),
            np.concatenate(cand_off).astype(np.int64), np.concatenate(cand_idx).astype(np.int64))


def field_env_writer(spec: FieldEnvSpec, clim: ClimateSpec, table_steps: int, occ_seed: int,
                     conv: ConvSpec | None = None) -> SbbWriter:
    """One FDM-scale env scenario: the plan's field sections (fdm.fdm_writer,
    with its rooms' cells and area-weighted air-side columns), stochastic
    convection off or, with `conv`, on in every room (the shipped buildings
    all carry p = 0.1, distance 2: data/blob_meta/*.json "conv"), and
    hvac_sections with the rooms as zones (zone area = the room's floor area,
    internal gains per cell of the plan's cell size). No solar gain section:
    the reference core has no solar input."""
    from .fdm import fdm_writer, make_plan

    plan = make_plan(spec.field)
    w = fdm_writer(plan)
    Z = plan.k
    b = make_building(Z, spec.ahus, spec.seed, name=spec.name)
    if conv is None:
        w.scalar_f64("conv_p", 0.0)
        w.scalar_f64("conv_distance", 0.0)
        w.scalar_i64("conv_seed", 0)
        w.add("conv_room_offsets", [0], "i32")
        w.add("conv_room_cells", np.zeros(0), "i32")
        w.add("conv_cand_offsets", [0], "i32")
        w.add("conv_cand_idx", np.zeros(0), "i32")
    else:
        c_off, c_cells, c_coff, c_idx = field_conv_tables(plan, conv.distance)
        w.scalar_f64("conv_p", conv.p)
        w.scalar_f64("conv_distance", float(conv.distance))
        w.scalar_i64("conv_seed", conv.seed)
        w.add("conv_room_offsets", c_off, "i32")
        w.add("conv_room_cells", c_cells, "i32")
        w.add("conv_cand_offsets", c_coff, "i32")
        w.add("conv_cand_idx", c_idx, "i32")
    cv = spec.field.cv_m
    zone_area = np.array([c.size for c in plan.room_cells], np.float64) * cv * cv
    hvac_sections(w, b, Z, clim, table_steps, occ_seed, zone_area, cv * 100.0, None, None)
    return w
