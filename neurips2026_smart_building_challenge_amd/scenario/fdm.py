"""Seeded FDM-scale buildings: a 2-D finite-difference floor plan at the size
of the reference's shipped buildings, written as an SBB1 blob with the field
sections csim's sb_fdm reads (complete_port/csim/sb_fdm.c:40-118).

The reference's buildings are 123K-1.17M control volumes on a (rows, cols)
grid with 32-285 rooms (data/blob_meta/*.json; building_train_1 is 606 x 339 =
205,434 cells, 39 rooms, 3.13M nonzeros per LU factor). This generator draws
one such plan from a seed:

  - a margin of exterior cells (not solved: csim resets them to the ambient
    temperature every step, sb_fdm.c:186-187);
  - an exterior wall ring and 1-cell interior walls (concrete-like cells);
  - rooms from a seeded binary space partition of the interior (air cells with
    an effective mixing conductivity and interior mass);
  - conduction between 4-neighbour solved cells through the harmonic mean of
    their half-cell conductances; convective exposure of cells that face the
    exterior (ambient_face_areas_0/1, the h-dependent term of sb_fdm.c:126-140);
    a small Dirichlet loss per cell (roof and ground);
  - the air side of every room as general area-weighted columns: applied
    spreads a VAV's power over the room's cells (1 / cells each), sensed
    averages them (sb_fdm.c:104-118, 155-181 read them as sparse columns);
  - the system A = diag(cap + dirichlet + exposure(h0) + mass coupling) + the
    conduction Laplacian, factorized by scipy's SuperLU with the reference
    baker's options (complete_port/pysim/bake_scenario.py:131-135:
    permc_spec="MMD_AT_PLUS_A", default pivoting), baked as CSC L / U and the
    row / column permutations, plus the baker's reference solve
    (solref_b / solref_x, bake_scenario.py:138-143).

Cell p = r * cols + c; solved cells are listed in ascending p.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from .sbb import SbbWriter

T0 = 273.15
DT_SEC = 300.0
HEIGHT = 3.0              # m, storey height: every face is d x HEIGHT
H0 = 8.8                  # W/m^2K, the blob's convection coefficient (the baked system's h)


@dataclass(frozen=True)
class FdmSpec:
    rows: int = 606
    cols: int = 339
    rooms: int = 39
    margin: int = 30          # exterior cells around the footprint
    wall: int = 2             # exterior wall thickness (cells)
    cv_m: float = 0.3         # cell edge (m)
    seed: int = 1

    @property
    def name(self) -> str:
        return f"fdm_{self.rows}x{self.cols}_r{self.rooms}_s{self.seed}"


@dataclass
class FdmPlan:
    spec: FdmSpec
    kind: np.ndarray          # (rows, cols) int8: -1 exterior, 0 wall, 1 room air
    room: np.ndarray          # (rows, cols) int32 room index or -1
    solved: np.ndarray        # (n,) int64 cell ids
    A: "object"               # scipy.sparse csc (n, n)
    cap: np.ndarray
    dirichlet: np.ndarray
    mass_coupling: np.ndarray
    mass_retained: np.ndarray
    mass_gained: np.ndarray
    horizontal: np.ndarray    # (n_cvs,) m
    vertical: np.ndarray      # (n_cvs,) m
    conductivity: np.ndarray  # (n_cvs,) W/mK
    face0: np.ndarray         # (n_cvs,) m^2 facing the exterior along a row
    face1: np.ndarray         # (n_cvs,) m^2 facing the exterior along a column
    temp_init: np.ndarray     # (n_cvs,)
    mass_temp_init: np.ndarray
    room_cells: list          # per room: solved indices t (ascending)

    @property
    def n(self) -> int:
        return int(self.solved.size)

    @property
    def n_cvs(self) -> int:
        return self.spec.rows * self.spec.cols

    @property
    def k(self) -> int:
        return len(self.room_cells)


def _partition(rng: np.random.Generator, r0: int, c0: int, r1: int, c1: int, count: int) -> list:
    """Splits [r0, r1) x [c0, c1) into `count` rectangles separated by 1-cell
    walls: the largest piece is cut across its longer side at a seeded
    fraction until there are `count` pieces."""
    pieces = [(r0, c0, r1, c1)]
    while len(pieces) < count:
        areas = [(a[2] - a[0]) * (a[3] - a[1]) for a in pieces]
        i = int(np.argmax(areas))
        a0, b0, a1, b1 = pieces.pop(i)
        h, w = a1 - a0, b1 - b0
        f = rng.uniform(0.35, 0.65)
        if h >= w:
            cut = a0 + max(3, min(h - 4, int(round(h * f))))
            pieces += [(a0, b0, cut, b1), (cut + 1, b0, a1, b1)]
        else:
            cut = b0 + max(3, min(w - 4, int(round(w * f))))
            pieces += [(a0, b0, a1, cut), (a0, cut + 1, a1, b1)]
    return sorted(pieces)


def exposure(plan: FdmPlan, h: float) -> np.ndarray:
    """Per solved cell, sb_fdm.c:126-140 (same operation order)."""
    p = plan.solved
    out = np.zeros(plan.n)
    a0, a1 = plan.face0[p], plan.face1[p]
    hz, vt, cd = plan.horizontal[p], plan.vertical[p], plan.conductivity[p]
    m0, m1 = a0 > 0.0, a1 > 0.0
    out[m0] += h * a0[m0] / (1.0 + h * 0.5 * hz[m0] / cd[m0])
    out[m1] += h * a1[m1] / (1.0 + h * 0.5 * vt[m1] / cd[m1])
    return out


def make_plan(spec: FdmSpec) -> FdmPlan:
    import scipy.sparse as sp

    rng = np.random.default_rng(spec.seed)
    R, C, d = spec.rows, spec.cols, spec.cv_m
    m, wt = spec.margin, spec.wall
    if R - 2 * (m + wt) < 8 or C - 2 * (m + wt) < 8:
        raise ValueError("grid too small for its margin and walls")
    kind = np.full((R, C), -1, np.int8)
    kind[m:R - m, m:C - m] = 0
    room = np.full((R, C), -1, np.int32)
    for i, (a0, b0, a1, b1) in enumerate(_partition(rng, m + wt, m + wt, R - m - wt, C - m - wt, spec.rooms)):
        kind[a0:a1, b0:b1] = 1
        room[a0:a1, b0:b1] = i
    flat = kind.reshape(-1)
    solved = np.flatnonzero(flat >= 0).astype(np.int64)
    n = solved.size
    idx = np.full(R * C, -1, np.int64)
    idx[solved] = np.arange(n)
    idx2 = idx.reshape(R, C)

    # per-cell material (walls: concrete-like; rooms: air with an effective
    # mixing conductivity), jittered per cell
    jit = rng.uniform(0.95, 1.05, size=(R, C))
    k_cell = np.where(kind == 1, 2.0, 1.4) * jit
    rho_c = np.where(kind == 1, 1.2 * 1005.0 * 3.0, 2.0e6) * jit   # J/m^3K (air: furniture-free volume x 3)
    vol = d * d * HEIGHT
    conductivity = k_cell.reshape(-1).copy()
    conductivity[flat < 0] = 1.0
    horizontal = np.full(R * C, d)
    vertical = np.full(R * C, d)

    cap_cell = (rho_c * vol / DT_SEC).reshape(-1)
    cap = cap_cell[solved]
    dirichlet = np.full(n, 0.3 * d * d)            # roof / ground loss, W/K
    # faces to the exterior (a solved cell next to an exterior cell)
    ext = kind < 0
    face0 = np.zeros((R, C))
    face1 = np.zeros((R, C))
    inside = kind >= 0
    for dc in (-1, 1):
        nb = np.zeros_like(ext)
        if dc < 0:
            nb[:, 1:] = ext[:, :-1]
        else:
            nb[:, :-1] = ext[:, 1:]
        face0 += np.where(inside & nb, d * HEIGHT, 0.0)
    for dr in (-1, 1):
        nb = np.zeros_like(ext)
        if dr < 0:
            nb[1:, :] = ext[:-1, :]
        else:
            nb[:-1, :] = ext[1:, :]
        face1 += np.where(inside & nb, d * HEIGHT, 0.0)
    face0 = face0.reshape(-1)
    face1 = face1.reshape(-1)

    # interior mass on room air cells
    air = flat[solved] == 1
    gm = 4.0 * d * d
    cm = 25e3 * d * d
    ret = math.exp(-gm * DT_SEC / cm)
    mc = np.where(air, gm, 0.0)
    mret = np.where(air, ret, 1.0)
    mgain = np.where(air, 1.0 - ret, 0.0)

    # conduction between 4-neighbour solved cells (harmonic half-cell resistances)
    rows_i, cols_i, vals = [], [], []
    diag = np.zeros(n)
    for dr, dc in ((0, 1), (1, 0)):
        a = idx2[:R - dr, :C - dc]
        b = idx2[dr:, dc:]
        ka = k_cell[:R - dr, :C - dc]
        kb = k_cell[dr:, dc:]
        ok = (a >= 0) & (b >= 0)
        a, b = a[ok], b[ok]
        g = (d * HEIGHT) / (0.5 * d / ka[ok] + 0.5 * d / kb[ok])
        rows_i += [a, b]
        cols_i += [b, a]
        vals += [-g, -g]
        np.add.at(diag, a, g)
        np.add.at(diag, b, g)
    plan = FdmPlan(spec, kind, room, solved, None, cap, dirichlet, mc, mret, mgain, horizontal, vertical,
                   conductivity, face0, face1, np.zeros(R * C), np.zeros(n), [])
    diag += cap + dirichlet + exposure(plan, H0) + mc
    rows_i.append(np.arange(n))
    cols_i.append(np.arange(n))
    vals.append(diag)
    A = sp.csc_matrix((np.concatenate(vals), (np.concatenate(rows_i), np.concatenate(cols_i))), shape=(n, n))
    A.sum_duplicates()
    A.sort_indices()
    plan.A = A

    temp = np.full(R * C, T0 + 10.0)
    temp[solved] = T0 + 21.0 + rng.uniform(-0.5, 0.5, size=n)
    plan.temp_init = temp
    plan.mass_temp_init = np.where(mc > 0.0, temp[solved], 0.0)
    rflat = room.reshape(-1)[solved]
    plan.room_cells = [np.flatnonzero(rflat == i).astype(np.int64) for i in range(spec.rooms)]
    return plan


def fdm_writer(plan: FdmPlan) -> SbbWriter:
    """The field sections of one plan (the names and dtypes of the reference
    baker, bake_scenario.py:100-152)."""
    import scipy.sparse as sp
    import scipy.sparse.linalg as spla

    s = plan.spec
    n, k = plan.n, plan.k
    w = SbbWriter()
    w.add("grid", [s.rows, s.cols], "i64")
    w.add("solved", plan.solved, "i64")
    w.add("dirichlet_conductance", plan.dirichlet, "f64")
    w.add("capacitance_rate", plan.cap, "f64")
    w.add("mass_coupling", plan.mass_coupling, "f64")
    w.add("mass_retained", plan.mass_retained, "f64")
    w.add("mass_gained", plan.mass_gained, "f64")
    w.add("mass_temp_init", plan.mass_temp_init, "f64")
    w.add("temp_init", plan.temp_init, "f64")
    w.add("horizontal", plan.horizontal, "f64")
    w.add("vertical", plan.vertical, "f64")
    w.add("solver_conductivity", plan.conductivity, "f64")
    w.add("ambient_face_areas_0", plan.face0, "f64")
    w.add("ambient_face_areas_1", plan.face1, "f64")
    w.scalar_f64("convection_coefficient", H0)
    A = plan.A.tocsc()
    w.add("A_system_shape", [n, n], "i64")
    w.add("A_system_indptr", A.indptr, "i32")
    w.add("A_system_indices", A.indices, "i32")
    w.add("A_system_data", A.data, "f64")
    lu = spla.splu(A, permc_spec="MMD_AT_PLUS_A")
    L, U = lu.L.tocsc(), lu.U.tocsc()
    L.sort_indices()
    U.sort_indices()
    w.add("lu_perm_r", np.asarray(lu.perm_r, np.int32), "i32")
    w.add("lu_perm_c", np.asarray(lu.perm_c, np.int32), "i32")
    for name, M in (("lu_L", L), ("lu_U", U)):
        w.add(f"{name}_shape", [n, n], "i64")
        w.add(f"{name}_indptr", M.indptr, "i32")
        w.add(f"{name}_indices", M.indices, "i32")
        w.add(f"{name}_data", M.data, "f64")
    b = np.sin(0.1 * np.arange(n) + 1.0)
    w.add("solref_b", b, "f64")
    w.add("solref_x", lu.solve(b), "f64")
    # air side: room i's VAV applies its power spread over the room's cells and
    # senses their mean
    cnt = np.array([c.size for c in plan.room_cells], np.float64)
    ap_i = np.concatenate(plan.room_cells)
    ap_p = np.concatenate([[0], np.cumsum([c.size for c in plan.room_cells])])
    ap_x = np.concatenate([np.full(c.size, 1.0 / cnt[i]) for i, c in enumerate(plan.room_cells)])
    w.add("applied_shape", [n, k], "i64")
    w.add("applied_indptr", ap_p, "i32")
    w.add("applied_indices", ap_i, "i32")
    w.add("applied_data", ap_x, "f64")
    w.add("sensed_shape", [k, n], "i64")
    w.add("sensed_indptr", ap_p, "i32")
    w.add("sensed_indices", ap_i, "i32")
    w.add("sensed_data", ap_x, "f64")
    # the simulator's copy over all cells (n_cvs x k CSR: cell -> its room's column)
    rc = plan.room.reshape(-1)
    AS = sp.csr_matrix((np.ones(int((rc >= 0).sum())), (np.flatnonzero(rc >= 0), rc[rc >= 0])), shape=(s.rows * s.cols, k))
    w.add("air_side_sensed_shape", [s.rows * s.cols, k], "i64")
    w.add("air_side_sensed_indptr", AS.indptr, "i32")
    w.add("air_side_sensed_indices", AS.indices, "i32")
    w.add("air_side_sensed_data", AS.data, "f64")
    w.add("room_offsets", ap_p, "i32")
    rcell = plan.solved[ap_i]
    w.add("room_cells", np.stack([rcell // s.cols, rcell % s.cols], 1).reshape(-1), "i32")
    return w


def step_inputs(plan: FdmPlan, n_envs: int, seed: int, step: int) -> dict[str, np.ndarray]:
    """Seeded inputs of one batched field step: per env the heat per cell
    (each room's heat spread over its cells, as the env's zone heat is), the
    ambient temperature, h, and per room the air-side conductance (some zero,
    so both branches of the air-side test run) and supply temperature."""
    rng = np.random.default_rng([seed, step])
    n_cvs, k = plan.n_cvs, plan.k
    q = np.zeros((n_envs, n_cvs))
    heat = rng.uniform(-2000.0, 6000.0, size=(n_envs, k))
    for i, cells in enumerate(plan.room_cells):
        q[:, plan.solved[cells]] = (heat[:, i] / cells.size)[:, None]
    ambient = T0 + 8.0 + 10.0 * np.sin(2.0 * np.pi * step / 288.0) + rng.normal(0.0, 1.0, size=n_envs)
    h = np.where(rng.random(n_envs) < 0.5, H0, rng.uniform(4.0, 20.0, size=n_envs))
    g = rng.uniform(0.0, 400.0, size=(n_envs, k)) * (rng.random((n_envs, k)) < 0.8)
    g[0 if n_envs == 1 else 1, :] = 0.0 if step % 3 == 0 else g[0 if n_envs == 1 else 1, :]   # an env with no air side
    air_t = T0 + rng.uniform(12.0, 40.0, size=(n_envs, k))
    return {"input_q": q, "ambient": ambient, "h": h, "air_g": g, "air_T": air_t}
