"""ctypes front-end for the two CPU oracles (TEST INFRASTRUCTURE).

  OracleEnv : oracle/liboracle.so, this repo's C restatement of csim
  RefEnv    : oracle/_ref/libcsim_ref.so, the reference csim compiled from
              /root/reference (present only where that build ran)

Both expose the same per-env protocol (the reference CPU env's puf_reset /
puf_step, complete_port/pufferlib_cpu_env.h:187-257) and a threaded batch runner
used as the CPU baseline. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# SBENV_CONT_BIG=1: the SB_CONT_BIG action row (320 continuous slots), as the
# env library of the same process (libsbenv_big.so) lays it out
CONT_BIG = os.environ.get("SBENV_CONT_BIG", "0") not in ("", "0")
ORACLE_SO = HERE / ("liboracle_big.so" if CONT_BIG else "liboracle.so")
REF_SO = HERE / "_ref" / "libcsim_ref.so"
SB_OBS, SB_CONT, SB_DISC = 1024, (320 if CONT_BIG else 256), 16
P = ctypes.c_void_p


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(P)


class _Lib:
    def __init__(self, path: Path, prefix: str):
        self.lib = ctypes.CDLL(str(path))
        self.prefix = prefix
        L = self.lib
        if prefix == "ref":
            L.ref_open.restype = P
            L.ref_open.argtypes = [ctypes.c_char_p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int, ctypes.c_int]
            self.open_fn = L.ref_open
            self.close_fn = L.ref_close
            self.reset_fn, self.step_fn, self.state_fn = L.ref_reset, L.ref_step, L.ref_state
            self.batch_fn = L.ref_run_batch
            self.row_fn = L.ref_action_row
            L.ref_last_reward_f64.restype = ctypes.c_double
            L.ref_last_reward_f64.argtypes = [P]
            for f in (L.ref_obs_len, L.ref_n_cont, L.ref_n_disc, L.ref_n_cvs):
                f.argtypes = [P]
            L.ref_native.argtypes = [P, P]
            L.ref_parts.argtypes = [P, P]
            L.ref_log.argtypes = [P, P]
            L.ref_clear_log.argtypes = [P]
        else:
            L.sbo_scen_open.argtypes = [P, ctypes.c_char_p]
            L.sbo_scen_close.argtypes = [P]
            L.sbo_env_new.restype = P
            L.sbo_env_new.argtypes = [P, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int, ctypes.c_int]
            self.close_fn = L.sbo_env_free
            self.reset_fn, self.step_fn, self.state_fn = L.sbo_env_reset, L.sbo_env_step, L.sbo_env_state
            self.batch_fn = L.sbo_run_batch
            self.row_fn = L.sbo_action_row
            L.sbo_env_last_reward.argtypes = [P]
            L.sbo_env_last_reward.restype = ctypes.c_double
            for f in (L.sbo_env_obs_len, L.sbo_env_n_cont, L.sbo_env_n_disc):
                f.argtypes = [P]
            L.sbo_env_log.argtypes = [P, P]
            L.sbo_env_parts.argtypes = [P, P]
            L.sbo_env_set_first_steps.argtypes = [P, ctypes.c_int]
            L.sbo_mt_seed.argtypes = [P, ctypes.c_uint32]
            L.sbo_mt_u32.argtypes = [P]
            L.sbo_mt_u32.restype = ctypes.c_uint32
            L.sbo_mt_double.argtypes = [P]
            L.sbo_mt_double.restype = ctypes.c_double
            L.sbo_mt_interval.argtypes = [P, ctypes.c_uint32]
            L.sbo_mt_interval.restype = ctypes.c_uint32
        self.close_fn.argtypes = [P]
        self.reset_fn.argtypes = [P, P]
        self.step_fn.argtypes = [P, P, P, P, P]
        self.step_fn.restype = ctypes.c_int
        self.state_fn.argtypes = [P, P]
        self.state_fn.restype = ctypes.c_int
        self.batch_fn.argtypes = [P, P, ctypes.c_int, ctypes.c_int, ctypes.c_uint64, ctypes.c_int, P]
        self.batch_fn.restype = ctypes.c_double
        self.row_fn.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                                ctypes.c_int, ctypes.c_int, P]


_LIBS: dict[str, _Lib] = {}


def lib(kind: str) -> _Lib:
    if kind not in _LIBS:
        if kind == "ref" and CONT_BIG:
            raise RuntimeError("the reference core's driver lays out 256 continuous slots, not SB_CONT_BIG's 320")
        path = REF_SO if kind == "ref" else ORACLE_SO
        if not path.exists():
            raise FileNotFoundError(f"{path} is not built (run __graft_entry__.build())")
        _LIBS[kind] = _Lib(path, "ref" if kind == "ref" else "sbo")
    return _LIBS[kind]


def ref_available() -> bool:
    return REF_SO.exists() and not CONT_BIG


class _Scen:
    """Keeps one oracle scenario (SboScen) alive for the envs that share it."""

    SIZE = 65536

    def __init__(self, path: str):
        self.buf = ctypes.create_string_buffer(self.SIZE)
        L = lib("oracle").lib
        if L.sbo_scen_open(ctypes.addressof(self.buf), str(path).encode()) != 0:
            raise RuntimeError(f"oracle cannot open {path}")
        self.path = str(path)

    def __del__(self):
        try:
            lib("oracle").lib.sbo_scen_close(ctypes.addressof(self.buf))
        except Exception:
            pass


_SCEN_CACHE: dict[str, _Scen] = {}


def scenario(path) -> _Scen:
    key = str(path)
    if key not in _SCEN_CACHE:
        _SCEN_CACHE[key] = _Scen(key)
    return _SCEN_CACHE[key]


_SEEDS: dict[str, tuple[int, int]] = {}


_CAPS: dict[str, int] = {}


def _state_cap(path) -> int:
    """Doubles a state snapshot may hold: the field (every cell and the
    solved cells' interior mass) plus at most 8192 of HVAC state."""
    key = str(path)
    if key not in _CAPS:
        from neurips2026_smart_building_challenge_amd.scenario.sbb import read_sbb

        b = read_sbb(path)
        _CAPS[key] = int(np.prod(b["grid"])) + int(b["solved"].size) + 8192
    return _CAPS[key]


def default_conv_seed(path, occ_seed: int) -> int:
    """The convection stream seed of the env whose occupancy seed is occ_seed:
    the blob's conv_seed offset by the env's index within its scenario (the
    GPU vec seeds env j of a scenario with occ_seed + j and conv_seed + j)."""
    key = str(path)
    if key not in _SEEDS:
        from neurips2026_smart_building_challenge_amd.scenario.sbb import read_sbb

        b = read_sbb(path)
        _SEEDS[key] = (int(b["occ_seed"][0]), int(b["conv_seed"][0]))
    occ0, conv0 = _SEEDS[key]
    return (conv0 + int(occ_seed) - occ0) & 0xFFFFFFFF


class CpuEnv:
    """One env of either oracle, stepping with the reference CPU env protocol."""

    def __init__(self, kind: str, path, occ_seed: int, start: int = 0, max_steps: int = 8640,
                 conv_seed: int | None = None, first_steps: int | None = None):
        self.kind = kind
        self.L = lib(kind)
        if conv_seed is None:
            conv_seed = default_conv_seed(path, occ_seed)
        if kind == "ref":
            self.h = self.L.open_fn(str(path).encode(), occ_seed, conv_seed, start, max_steps)
            self.n_cont = self.L.lib.ref_n_cont(self.h)
            self.n_disc = self.L.lib.ref_n_disc(self.h)
        else:
            self.scen = scenario(path)
            self.h = self.L.lib.sbo_env_new(ctypes.addressof(self.scen.buf), occ_seed, conv_seed, start,
                                            max_steps)
            if self.h:
                self.n_cont = self.L.lib.sbo_env_n_cont(self.h)
                self.n_disc = self.L.lib.sbo_env_n_disc(self.h)
        if not self.h:
            raise RuntimeError(f"cannot open env on {path}")
        if first_steps is not None and first_steps != max_steps:
            if kind == "ref":
                raise ValueError("first-episode truncation is a GPU-env feature the reference CPU core lacks")
            self.L.lib.sbo_env_set_first_steps(self.h, int(first_steps))
        self.obs = np.zeros(SB_OBS, np.float32)
        self._r = np.zeros(1, np.float32)
        self._t = np.zeros(1, np.float32)
        self._st = np.zeros(_state_cap(path), np.float64)

    def close(self):
        if getattr(self, "h", None):
            self.L.close_fn(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def reset(self) -> np.ndarray:
        self.L.reset_fn(self.h, _ptr(self.obs))
        return self.obs.copy()

    def step(self, action_row: np.ndarray):
        a = np.ascontiguousarray(action_row, dtype=np.float32)
        done = self.L.step_fn(self.h, _ptr(a), _ptr(self.obs), _ptr(self._r), _ptr(self._t))
        return self.obs.copy(), float(self._r[0]), float(self._t[0]), bool(done)

    @property
    def obs_len(self) -> int:
        if self.kind == "ref":
            return int(self.L.lib.ref_obs_len(self.h))
        return int(self.L.lib.sbo_env_obs_len(self.h))

    def last_reward_f64(self) -> float:
        if self.kind == "ref":
            return float(self.L.lib.ref_last_reward_f64(self.h))
        return float(self.L.lib.sbo_env_last_reward(self.h))

    def log(self) -> np.ndarray:
        out = np.zeros(6, np.float32)
        if self.kind == "ref":
            self.L.lib.ref_log(self.h, _ptr(out))
        else:
            self.L.lib.sbo_env_log(self.h, _ptr(out))
        return out

    def state(self) -> np.ndarray:
        n = self.L.state_fn(self.h, _ptr(self._st))
        return self._st[:n].copy()

    def parts(self) -> np.ndarray:
        """The last step's reward parts: sb_reward's 12 (npr, nec, ncar, electricity
        and gas cost, blower, cooling, pump power, price, dt, hour, workday); the
        oracle adds the reference GPU env's comfort diagnostics (mean and worst
        zone deviation, out-of-band fraction) and the gas rate."""
        if self.kind == "ref":
            out = np.zeros(12, np.float64)
            self.L.lib.ref_parts(self.h, _ptr(out))
        else:
            out = np.zeros(16, np.float64)
            self.L.lib.sbo_env_parts(self.h, _ptr(out))
        return out


LOG_KEYS = ["perf", "score", "episode_return", "episode_length", "comfort_dev_K", "worst_dev_K", "out_of_band_frac",
            "productivity", "energy_cost_norm", "carbon_norm", "elec_kwh", "gas_kwh", "n"]


class GpuEnvLog:
    """The reference GPU env's episode log (complete_port/gpu/smart_buildings.cu:
    101-115, filled by finalize_k :1936-2047), replayed in float32 from an env's
    per-step float32 reward and the oracle's reward parts: running sums of the
    reward and of 8 diagnostics (productivity term, normalized cost, normalized
    carbon, mean zone deviation, the worst deviation as a maximum,
    out-of-band fraction, electricity and gas kWh), added to the Log when a full
    episode ends (a desync-cut first episode is dropped), then cleared."""

    def __init__(self):
        self.log = {k: np.float32(0.0) for k in LOG_KEYS}
        self.ret = np.float32(0.0)
        self.part = np.zeros(8, np.float32)
        self.worst = np.float32(0.0)

    @staticmethod
    def step_parts(pt: np.ndarray) -> np.ndarray:
        """The GPU env's 8 per-step diagnostics (sb_gpu_kernels.cuh:1466-1473) from the
        oracle's 16 parts."""
        dt = pt[9]
        elec = pt[5] + abs(pt[6]) + pt[7]
        return np.array([pt[0], pt[1], pt[2], pt[12], pt[13], pt[14], abs(elec) * dt / 3.6e6, pt[15] * dt / 3.6e6])

    def step(self, r: float, pt: np.ndarray, step: int, done: bool, cut: bool):
        f = np.float32
        rp = self.step_parts(pt)
        self.ret = f(self.ret + f(r))
        for k in range(8):
            self.part[k] = f(self.part[k] + f(rp[k]))
        if f(rp[4]) > self.worst:
            self.worst = f(rp[4])
        if not done:
            return
        if not cut:
            st = f(step)
            L = self.log
            mean = f(self.ret / st)
            L["perf"] = f(L["perf"] + mean)
            L["score"] = f(L["score"] + mean)
            L["episode_return"] = f(L["episode_return"] + self.ret)
            L["episode_length"] = f(L["episode_length"] + st)
            L["productivity"] = f(L["productivity"] + f(self.part[0] / st))
            L["energy_cost_norm"] = f(L["energy_cost_norm"] + f(self.part[1] / st))
            L["carbon_norm"] = f(L["carbon_norm"] + f(self.part[2] / st))
            L["comfort_dev_K"] = f(L["comfort_dev_K"] + f(self.part[3] / st))
            L["worst_dev_K"] = f(L["worst_dev_K"] + self.worst)
            L["out_of_band_frac"] = f(L["out_of_band_frac"] + f(self.part[5] / st))
            L["elec_kwh"] = f(L["elec_kwh"] + self.part[6])
            L["gas_kwh"] = f(L["gas_kwh"] + self.part[7])
            L["n"] = f(L["n"] + 1)
        self.ret = np.float32(0.0)
        self.part[:] = 0.0
        self.worst = np.float32(0.0)


CN_OBS, CN_ACT = 983, 219


class Canon:
    """The oracle's canonical layout of one blob (oracle/sbo_canon.c): the
    pid_water base controller, the canonical observation, the comfort guard
    and the residual / absolute action decode, one env and one step at a time."""

    def __init__(self, path):
        L = lib("oracle").lib
        L.sbo_canon_size.restype = ctypes.c_size_t
        L.sbo_canon_open.argtypes = [P, ctypes.c_char_p]
        L.sbo_canon_base.argtypes = [P, P, P, P, P]
        L.sbo_canon_features.argtypes = [P, P, P, P, P, P]
        L.sbo_canon_trust.argtypes = [P, P, ctypes.c_float, ctypes.c_float, ctypes.c_int, P]
        L.sbo_canon_decode.argtypes = [P, P, P, P, ctypes.c_int, ctypes.c_float, ctypes.c_float, P]
        self.L = L
        self.buf = ctypes.create_string_buffer(int(L.sbo_canon_size()))
        rc = L.sbo_canon_open(ctypes.addressof(self.buf), str(path).encode())
        if rc != 0:
            raise ValueError(f"canonical layout not available for {path} ({rc})")
        ints = np.frombuffer(self.buf, np.int32, count=4)
        self.K, self.n_act, self.n_cont, self.n_disc = (int(v) for v in ints)
        L.sbo_canon_slot.argtypes = [P, ctypes.c_int]
        self.slot_of_action = np.array([L.sbo_canon_slot(self._p(), i) for i in range(self.n_act)])

    def _p(self):
        return ctypes.addressof(self.buf)

    def base(self, obs: np.ndarray, pid: np.ndarray):
        """pid (float64 [18]) is updated in place; returns (base [n_act] float32, ahu_info [18] float32)."""
        o = np.ascontiguousarray(obs, np.float32)
        assert pid.dtype == np.float64 and pid.size >= 18 and pid.flags.c_contiguous
        base = np.zeros(self.n_act, np.float32)
        ai = np.zeros(18, np.float32)
        self.L.sbo_canon_base(self._p(), _ptr(o), _ptr(pid), _ptr(base), _ptr(ai))
        return base, ai

    def features(self, obs, base, ahu_info, pid) -> np.ndarray:
        o = np.ascontiguousarray(obs, np.float32)
        x = np.zeros(CN_OBS, np.float32)
        self.L.sbo_canon_features(self._p(), _ptr(o), _ptr(np.ascontiguousarray(base, np.float32)),
                                  _ptr(np.ascontiguousarray(ahu_info, np.float32)),
                                  _ptr(np.ascontiguousarray(pid, np.float64)), _ptr(x))
        return x

    def trust(self, obs, d0: float, d1: float, hot: int) -> np.ndarray:
        o = np.ascontiguousarray(obs, np.float32)
        w = np.zeros(self.n_act, np.float32)
        self.L.sbo_canon_trust(self._p(), _ptr(o), d0, d1, int(hot), _ptr(w))
        return w

    def decode(self, base, p_row, trust, resid: int, scale: float, dscale: float) -> np.ndarray:
        """The native action row (272 floats) the env step decodes."""
        row = np.zeros(SB_CONT + SB_DISC, np.float32)
        pr = np.zeros(SB_CONT + SB_DISC, np.float32)
        pr[:len(p_row)] = p_row
        tr = None if trust is None else np.ascontiguousarray(trust, np.float32)
        self.L.sbo_canon_decode(self._p(), _ptr(np.ascontiguousarray(base, np.float32)), _ptr(pr),
                                _ptr(tr) if tr is not None else None, int(resid), scale, dscale, _ptr(row))
        return row


def desync_first_steps(env_index: int, episode_steps: int) -> int:
    """Length of env `env_index`'s first episode under the GPU env's desync
    (complete_port/gpu/smart_buildings.cu:2808-2815): a splitmix-style hash of
    the env index mapped into [1, episode_steps]."""
    m = (1 << 64) - 1
    h = (0x9E3779B97F4A7C15 * (env_index + 1)) & m
    h ^= h >> 31
    h = (h * 0xBF58476D1CE4E5B9) & m
    h ^= h >> 29
    return 1 + h % episode_steps


def action_row(seed: int, env: int, step: int, n_cont: int, n_disc: int, kind: str = "oracle") -> np.ndarray:
    row = np.zeros(SB_CONT + SB_DISC, np.float32)
    lib(kind).row_fn(seed, env, step, n_cont, n_disc, _ptr(row))
    return row


def run_batch(envs: list[CpuEnv], env_ids, steps: int, seed: int, nthreads: int) -> tuple[float, float]:
    """Steps every env `steps` times on `nthreads` threads; returns (seconds, reward_sum)."""
    kind = envs[0].kind
    arr = (P * len(envs))(*[e.h for e in envs])
    ids = np.ascontiguousarray(env_ids, dtype=np.int32)
    acc = np.zeros(1, np.float64)
    secs = lib(kind).batch_fn(ctypes.cast(arr, P), _ptr(ids), len(envs), steps, seed, nthreads, _ptr(acc))
    return float(secs), float(acc[0])


class Fdm:
    """The building-scale field model alone, G envs of one blob:
    kind "oracle" is this repo's restatement (sbo_fdm.c), kind "ref" the
    reference core's sb_fdm (oracle/_ref). Fields are host arrays: T (G, n_cvs),
    M (G, n_solved)."""

    def __init__(self, kind: str, path, G: int):
        self.kind, self.G = kind, G
        L = lib(kind).lib
        self.L = L
        dims = np.zeros(5, np.int32)
        if kind == "ref":
            L.ref_fdm_open.restype = P
            L.ref_fdm_open.argtypes = [ctypes.c_char_p, ctypes.c_int]
            for f in (L.ref_fdm_dims, L.ref_fdm_sensed_response):
                f.argtypes = [P, P]
            L.ref_fdm_lu_solve.argtypes = [P, P, P]
            L.ref_fdm_get.argtypes = [P, ctypes.c_int, P, P]
            L.ref_fdm_set.argtypes = [P, ctypes.c_int, P, P]
            L.ref_fdm_step_batch.argtypes = [P, P, P, P, P, P]
            L.ref_fdm_close.argtypes = [P]
            self.h = L.ref_fdm_open(str(path).encode(), G)
            if not self.h:
                raise RuntimeError(f"ref_fdm_open failed for {path}")
            L.ref_fdm_dims(self.h, _ptr(dims))
        else:
            L.sbo_fdm_open.restype = P
            L.sbo_fdm_open.argtypes = [ctypes.c_char_p]
            L.sbo_fdm_dims.argtypes = [P, P]
            L.sbo_fdm_sensed_response.restype = ctypes.POINTER(ctypes.c_double)
            L.sbo_fdm_sensed_response.argtypes = [P]
            L.sbo_fdm_init_state.argtypes = [P, P, P]
            L.sbo_fdm_lu_solve.argtypes = [P, P, P]
            L.sbo_fdm_step_batch.argtypes = [P, ctypes.c_int, P, P, P, P, P, P, P]
            L.sbo_fdm_step_batch.restype = ctypes.c_int
            L.sbo_fdm_close.argtypes = [P]
            self.h = L.sbo_fdm_open(str(path).encode())
            if not self.h:
                raise RuntimeError(f"sbo_fdm_open failed for {path}")
            L.sbo_fdm_dims(self.h, _ptr(dims))
        self.n_cvs, self.n, self.k, self.rows, self.cols = (int(x) for x in dims)
        if kind == "oracle":
            self.T = np.zeros((G, self.n_cvs))
            self.M = np.zeros((G, self.n))
            for g in range(G):
                L.sbo_fdm_init_state(self.h, _ptr(self.T[g]), _ptr(self.M[g]))

    def close(self):
        if self.h:
            (self.L.ref_fdm_close if self.kind == "ref" else self.L.sbo_fdm_close)(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def sensed_response(self) -> np.ndarray:
        if self.kind == "ref":
            out = np.zeros(self.k * self.k)
            self.L.ref_fdm_sensed_response(self.h, _ptr(out))
            return out.reshape(self.k, self.k)
        p = self.L.sbo_fdm_sensed_response(self.h)
        return np.ctypeslib.as_array(p, (self.k * self.k,)).copy().reshape(self.k, self.k)

    def lu_solve(self, b: np.ndarray) -> np.ndarray:
        b = np.ascontiguousarray(b, np.float64)
        x = np.zeros(self.n)
        (self.L.ref_fdm_lu_solve if self.kind == "ref" else self.L.sbo_fdm_lu_solve)(self.h, _ptr(b), _ptr(x))
        return x

    def state(self) -> tuple[np.ndarray, np.ndarray]:
        if self.kind == "oracle":
            return self.T.copy(), self.M.copy()
        T = np.zeros((self.G, self.n_cvs))
        M = np.zeros((self.G, self.n))
        for g in range(self.G):
            self.L.ref_fdm_get(self.h, g, _ptr(T[g]), _ptr(M[g]))
        return T, M

    def set_state(self, T: np.ndarray, M: np.ndarray):
        T = np.ascontiguousarray(T, np.float64)
        M = np.ascontiguousarray(M, np.float64)
        if self.kind == "oracle":
            self.T[...] = T
            self.M[...] = M
            return
        for g in range(self.G):
            self.L.ref_fdm_set(self.h, g, _ptr(T[g]), _ptr(M[g]))

    def step(self, inp: dict):
        q = np.ascontiguousarray(inp["input_q"], np.float64)
        amb = np.ascontiguousarray(inp["ambient"], np.float64)
        h = np.ascontiguousarray(inp["h"], np.float64)
        g = np.ascontiguousarray(inp["air_g"], np.float64)
        t = np.ascontiguousarray(inp["air_T"], np.float64)
        if self.kind == "ref":
            self.L.ref_fdm_step_batch(self.h, _ptr(q), _ptr(amb), _ptr(h), _ptr(g), _ptr(t))
        elif self.L.sbo_fdm_step_batch(self.h, self.G, _ptr(self.T), _ptr(self.M), _ptr(q), _ptr(amb), _ptr(h),
                                       _ptr(g), _ptr(t)) != 0:
            raise MemoryError("sbo_fdm_step_batch")
