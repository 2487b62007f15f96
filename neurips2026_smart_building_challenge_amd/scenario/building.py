"""Synthetic 2-floor RC buildings expressed in csim's data model.

A layout is `Z` zones on two floors of a rows x cols grid, served by `A` air
handlers. Every zone is one room with one control volume, and contributes three
thermal nodes to a (3, Z) grid:

  row 0  zone air        (the room cell; VAV supply air couples here)
  row 1  wall node       (exterior + partition walls of the zone)
  row 2  slab node       (floor/ceiling slab; ground on floor 0, roof on floor 1)

so cell p = row * Z + z, every cell is solved (solved[t] = t) and N = 3Z.
Conductances: air-wall, air-slab, wall-wall between horizontally adjacent zones,
slab-slab between a floor-0 zone and the zone above it, wall/air/slab to ambient
(Dirichlet), plus a west-to-east advective airflow between neighbouring zones of
a row. The advective term is upwind (only the downstream row gets the
off-diagonal), so A is non-symmetric but strictly diagonally dominant by rows.

Zone-air furniture mass uses csim's interior-mass terms (mass_coupling,
mass_retained, mass_gained; complete_port/csim/sb_fdm.c:146-152,183-185), and its
coupling conductance sits on A's diagonal, as in the reference's A_system
(complete_port/pysim/bake_scenario.py:125-131).

Sizes follow the hot-path contract: one VAV per zone, all VAVs air-side coupled
(k = Z), n_cont = 2Z + 3A + 2 and n_disc = A + 1 actions
(complete_port/pysim/bake_env.py:163-187 routing), n_dev = 6Z + 10A + 7
device observation fields (bake_env.py:228-268 id maps) and 7 auxiliary fields.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

RHO_AIR = 1.2
CP_AIR = 1006.0
DT_SEC = 300.0
T0 = 273.15

# device kinds and measurement ids of the observation map (bake_env.py:228-248)
AHU_FIELDS = 10   # ids 0..9
VAV_FIELDS = 6    # ids 0..5
HWS_FIELDS = 7    # ids 0..6
N_AUX = 7         # hod cos/sin, dow cos/sin, comfort now/soon, occupants

# Observation field names (the env's field_names, bake_env.py:112-113): device
# fields are "<device>_<measurement>", one measurement name per id of the maps
# at bake_env.py:228-250 (where two names share an id, the sensor's).
AHU_MEAS = ["cooling_request_count", "supply_air_static_pressure_sensor", "supply_air_flowrate_sensor",
            "supply_air_temperature_setpoint", "supply_fan_run_command", "supply_fan_speed_percentage_command",
            "outside_air_flowrate_sensor", "supervisor_run_command", "recirculation_percentage_command",
            "outside_air_temperature_sensor"]
VAV_MEAS = ["reheat_valve_percentage_command", "supply_air_damper_percentage_command",
            "supply_air_flowrate_setpoint", "zone_air_cooling_temperature_setpoint_sensor",
            "zone_air_heating_temperature_setpoint_sensor", "zone_air_temperature_sensor"]
HWS_MEAS = ["differential_pressure_setpoint", "supply_water_temperature_sensor", "differential_pressure_sensor",
            "supervisor_run_command", "heating_request_count", "run_status", "supply_water_temperature_setpoint"]
AUX_NAMES = ["hod_cos_000", "hod_sin_000", "dow_cos_000", "dow_sin_000", "comfort_mode_now", "comfort_mode_soon",
             "num_occupants"]


def field_name(kind: int, idx: int, obs_id: int) -> str:
    if kind == 2:
        return "hws_" + HWS_MEAS[obs_id]
    if kind == 0:
        return f"ahs_ahu_{idx + 1}_" + AHU_MEAS[obs_id]
    return f"VAV_{idx + 1}_" + VAV_MEAS[obs_id]


@dataclass
class Building:
    name: str
    n_zones: int
    n_ahu: int
    floors: int
    rows: int
    cols: int
    zone_pos: np.ndarray          # (Z, 3) floor,row,col
    zone_area: np.ndarray         # (Z,) m^2
    # thermal network (unknown t == cell p)
    cap_rate: np.ndarray          # C/dt, (N,)
    dirichlet: np.ndarray         # (N,)
    mass_coupling: np.ndarray     # (N,)
    mass_retained: np.ndarray     # (N,)
    mass_gained: np.ndarray       # (N,)
    A: "object"                   # scipy.sparse csc (N, N), the factorised system
    solar_coeff: np.ndarray       # (N,) m^2: q_solar = coeff * irradiance
    temp_init: np.ndarray         # (N,)
    mass_temp_init: np.ndarray    # (N,)
    # HVAC
    vav_ahu: np.ndarray           # (Z,) ahu index of vav v (= zone v)
    ahu_const: np.ndarray         # (A, 9)
    vav_const: np.ndarray         # (Z, 9)
    boiler_const: np.ndarray      # (10,)
    pump_const: np.ndarray        # (2,)
    header_res: float
    internal_w_m2: float
    standby_frac: float
    occupant_w: float
    cv_size_cm: float
    # action routing
    act_kind: np.ndarray
    act_index: np.ndarray
    act_actuator: np.ndarray
    act_is_disc: np.ndarray
    act_min_native: np.ndarray
    act_max_native: np.ndarray
    # observation map
    f_dev_kind: np.ndarray
    f_dev_idx: np.ndarray
    f_obs_id: np.ndarray
    f_norm_mean: np.ndarray
    f_norm_var: np.ndarray
    extra: dict = field(default_factory=dict)

    @property
    def n_nodes(self) -> int:
        return 3 * self.n_zones


def grid_shape(zones_per_floor: int) -> tuple[int, int]:
    rows = 3 if zones_per_floor <= 27 else 4
    cols = -(-zones_per_floor // rows)
    return rows, cols


def make_building(n_zones: int, n_ahu: int, seed: int, name: str | None = None) -> Building:
    """Builds one seeded layout. All geometry/parameter draws use `seed`."""
    import scipy.sparse as sp

    if n_zones < 2 or n_ahu < 1 or n_ahu > n_zones:
        raise ValueError("bad layout size")
    rng = np.random.default_rng(seed)
    Z, A = n_zones, n_ahu
    n0 = -(-Z // 2)
    per_floor = [n0, Z - n0]
    rows, cols = grid_shape(n0)
    widths = rng.uniform(5.0, 9.0, size=cols)     # m, per column
    depths = rng.uniform(5.0, 8.0, size=rows)     # m, per row
    height = 3.0

    pos = []
    slot = {}
    for f in range(2):
        for i in range(per_floor[f]):
            r, c = divmod(i, cols)
            slot[(f, r, c)] = len(pos)
            pos.append((f, r, c))
    pos = np.asarray(pos, dtype=np.int64)
    area = np.array([widths[c] * depths[r] for (_, r, c) in pos])

    N = 3 * Z
    air = np.arange(Z)
    wall = Z + np.arange(Z)
    slab = 2 * Z + np.arange(Z)

    cap = np.zeros(N)
    dirc = np.zeros(N)
    solar = np.zeros(N)
    rows_i: list[int] = []
    cols_i: list[int] = []
    vals: list[float] = []

    def couple(i: int, j: int, g: float) -> None:
        rows_i.extend([i, j, i, j])
        cols_i.extend([i, j, j, i])
        vals.extend([g, g, -g, -g])

    for z, (f, r, c) in enumerate(pos):
        a_fl = area[z]
        w, d = widths[c], depths[r]
        ext_len = 0.0
        if r == 0:
            ext_len += w
        if (f, r + 1, c) not in slot:
            ext_len += w
        if c == 0:
            ext_len += d
        if (f, r, c + 1) not in slot:
            ext_len += d
        part_len = 2.0 * (w + d) - ext_len
        ext_area = ext_len * height
        win = 0.4 * ext_area
        opaque = ext_area - win
        part_area = part_len * height
        jit = rng.uniform(0.9, 1.1, size=6)

        cap[air[z]] = RHO_AIR * CP_AIR * a_fl * height * 3.0 * jit[0] / DT_SEC
        cap[wall[z]] = (opaque * 120e3 + part_area * 25e3) * jit[1] / DT_SEC
        cap[slab[z]] = a_fl * 180e3 * jit[2] / DT_SEC
        # ambient couplings (W/K)
        infil = 0.3 * a_fl * height * RHO_AIR * CP_AIR / 3600.0
        dirc[air[z]] += 2.0 * win + infil
        dirc[wall[z]] += opaque / (1.0 + 0.05) * 0.9 * jit[3]
        dirc[slab[z]] += a_fl * (0.2 if f == 0 else 0.35) * jit[4]
        # surface couplings
        couple(air[z], wall[z], 3.0 * (ext_area + part_area))
        couple(air[z], slab[z], 3.0 * a_fl * jit[5])
        # solar: transmitted through windows to the air, absorbed fraction on
        # opaque walls, roof gain on the top floor slab
        solar[air[z]] = 0.4 * win * 0.5
        solar[wall[z]] = 0.6 * opaque * 0.04
        if f == 1:
            solar[slab[z]] = 0.7 * a_fl * 0.03

    # horizontal neighbours: shared partition walls + west->east airflow
    adv = np.zeros(N)
    adv_rows: list[int] = []
    adv_cols: list[int] = []
    adv_vals: list[float] = []
    for (f, r, c), z in slot.items():
        for (dr, dc) in ((0, 1), (1, 0)):
            zn = slot.get((f, r + dr, c + dc))
            if zn is None:
                continue
            shared = depths[r] if dc else widths[c]
            couple(wall[z], wall[zn], 1.5 * shared * height)
        east = slot.get((f, r, c + 1))
        mcp = 12.0 + 6.0 * rng.random()   # W/K
        if c == 0:
            dirc[air[z]] += mcp           # inflow from outdoors at the row head
        if east is not None:
            # zone `east` receives air at T_z: C dT_e/dt = mcp (T_z - T_e)
            adv[air[east]] += mcp
            adv_rows.append(air[east])
            adv_cols.append(air[z])
            adv_vals.append(-mcp)
        # vertical: slab of floor 0 under the floor-1 zone above
        if f == 0:
            up = slot.get((1, r, c))
            if up is not None:
                couple(slab[z], slab[up], 2.0 * area[z])

    # furniture mass on zone air
    mc = np.zeros(N)
    mret = np.ones(N)
    mgain = np.zeros(N)
    for z in range(Z):
        gm = 4.0 * area[z]                            # W/K
        cm = 25e3 * area[z]                           # J/K
        ret = math.exp(-gm * DT_SEC / cm)
        mc[air[z]] = gm
        mret[air[z]] = ret
        mgain[air[z]] = 1.0 - ret

    diag = cap + dirc + mc + adv
    rows_i.extend(range(N))
    cols_i.extend(range(N))
    vals.extend(diag.tolist())
    rows_i.extend(adv_rows)
    cols_i.extend(adv_cols)
    vals.extend(adv_vals)
    Am = sp.coo_matrix((vals, (rows_i, cols_i)), shape=(N, N)).tocsc()
    Am.sum_duplicates()
    Am.sort_indices()

    temp_init = np.full(N, T0 + 21.0) + rng.uniform(-0.5, 0.5, size=N)
    mass_init = np.where(mc > 0, temp_init, 0.0)

    # ---- HVAC ----
    bounds = [round(a * Z / A) for a in range(A + 1)]
    vav_ahu = np.zeros(Z, dtype=np.int32)
    for a in range(A):
        vav_ahu[bounds[a]:bounds[a + 1]] = a
    vav_const = np.zeros((Z, 9))
    for v in range(Z):
        vav_const[v] = [
            0.006 * area[v],            # max air flow m^3/s
            0.4 + 0.01 * area[v],       # reheat water flow factor (Kv)
            0.15,                       # min damper
            T0 + 45.0,                  # max discharge air temperature
            500.0,                      # static pressure at max flow (Pa)
            T0 + 21.0, T0 + 24.0,       # heating / cooling setpoints
            0.5, 0.0,                   # initial damper / reheat
        ]
    ahu_const = np.zeros((A, 9))
    for a in range(A):
        served = vav_ahu == a
        ahu_const[a] = [
            0.7,                                   # initial recirculation
            0.8 * vav_const[served, 0].sum(),      # max air flow
            100.0,                                 # min supply static pressure
            0.9,                                   # max recirculation
            3.5,                                   # cooling COP
            0.65,                                  # fan efficiency
            T0 + 13.0,                             # initial supply air temp
            400.0,                                 # initial static pressure
            1.0,                                   # initial run command
        ]
    boiler_const = np.array([T0 + 65.0, T0 + 50.0, 0.5, 0.25, 5.0,
                             2.0, 0.6, 1.5, 0.05, 0.05])
    pump_const = np.array([10.0, 0.7])

    # ---- actions: per AHU sat/static/recirc/run, HWS, per VAV damper+reheat ----
    # (the order of the competition env's action names: the discrete actions
    # are the AHU run commands in AHU order, then the hot-water run command,
    # which its baseline controllers index by position)
    kind, idx, act, disc, amin, amax = [], [], [], [], [], []

    def add_act(k, i, a, d, lo, hi):
        kind.append(k); idx.append(i); act.append(a); disc.append(d)
        amin.append(lo); amax.append(hi)

    for a in range(A):
        add_act(0, a, 0, 0, T0 + 12.0, T0 + 24.0)  # supply air temperature setpoint
        add_act(0, a, 1, 0, 100.0, 1000.0)         # static pressure setpoint
        add_act(0, a, 2, 0, 0.0, 1.0)              # recirculation command
        add_act(0, a, 3, 1, 0.0, 1.0)              # run command
    add_act(2, 0, 0, 0, T0 + 35.0, T0 + 75.0)     # supply water temperature setpoint
    add_act(2, 0, 1, 0, 0.3, 2.0)                 # differential pressure setpoint (bar)
    add_act(2, 0, 2, 1, 0.0, 1.0)                 # HWS run
    for v in range(Z):
        add_act(1, v, 0, 0, 0.0, 1.0)              # damper command
        add_act(1, v, 1, 0, 0.0, 1.0)              # reheat valve command

    # ---- observation map ----
    fk, fi, fo, fm, fv = [], [], [], [], []
    hws_norm = [(1.0, 0.2), (T0 + 60.0, 60.0), (1.0, 0.2), (0.9, 0.09),
                (float(Z), 0.0), (0.9, 0.09), (T0 + 55.0, 100.0)]
    for i, (m, s2) in enumerate(hws_norm):
        fk.append(2); fi.append(0); fo.append(i); fm.append(m); fv.append(s2)
    # one (mean, variance) per measurement name, as the env's normalizer keeps
    # them (bake_env.py:125-131), from the building's average air handler
    nserv = Z / A
    mflow = float(ahu_const[:, 1].mean())
    ahu_norm = [(nserv / 2.0, nserv * nserv / 8.0), (400.0, 4.0e4), (0.5 * mflow, 0.1 * mflow ** 2),
                (T0 + 15.0, 9.0), (0.9, 0.09), (0.5, 0.08), (0.15 * mflow, 0.02 * mflow ** 2),
                (0.9, 0.09), (0.6, 0.06), (T0 + 10.0, 120.0)]
    for a in range(A):
        for i, (m, s2) in enumerate(ahu_norm):
            fk.append(0); fi.append(a); fo.append(i); fm.append(m); fv.append(s2)
    for v in range(Z):
        vav_norm = [(0.3, 0.1), (0.5, 0.08), (vav_const[v, 0], 0.0),
                    (T0 + 24.0, 4.0), (T0 + 20.0, 4.0), (T0 + 21.5, 6.0)]
        for i, (m, s2) in enumerate(vav_norm):
            fk.append(1); fi.append(v); fo.append(i); fm.append(m); fv.append(s2)

    return Building(
        name=name or f"rc{Z}z{A}a",
        n_zones=Z, n_ahu=A, floors=2, rows=rows, cols=cols,
        zone_pos=pos, zone_area=area,
        cap_rate=cap, dirichlet=dirc, mass_coupling=mc, mass_retained=mret,
        mass_gained=mgain, A=Am, solar_coeff=solar, temp_init=temp_init,
        mass_temp_init=mass_init,
        vav_ahu=vav_ahu, ahu_const=ahu_const, vav_const=vav_const,
        boiler_const=boiler_const, pump_const=pump_const, header_res=0.002,
        internal_w_m2=8.0, standby_frac=0.3, occupant_w=110.0, cv_size_cm=800.0,
        act_kind=np.asarray(kind, np.uint8), act_index=np.asarray(idx, np.int32),
        act_actuator=np.asarray(act, np.uint8), act_is_disc=np.asarray(disc, np.uint8),
        act_min_native=np.asarray(amin), act_max_native=np.asarray(amax),
        f_dev_kind=np.asarray(fk, np.uint8), f_dev_idx=np.asarray(fi, np.int32),
        f_obs_id=np.asarray(fo, np.uint8), f_norm_mean=np.asarray(fm),
        f_norm_var=np.asarray(fv),
    )
