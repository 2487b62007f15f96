"""FDM-scale scenarios behind the PufferLib ABI (puf_vec_create / puf_reset /
puf_step on a blob whose field is an FDM plan: csrc/field_env*.{h,cpp,hip}
around the field group of csrc/fdm*), against the oracle's env
(oracle/sbo_core.c, pinned to the reference core by tests/test_field_env_oracle.py)
and the reference core's fixture (tests/golden/field_env.json):

  - exact field mode (env.field_exact = 1): observations, float32 rewards,
    terminals and the full state (field, interior mass, HVAC state, air side,
    occupancy, plant) bit-identical to the oracle after every step, through an
    auto-reset, for three envs of one scenario (their occupancy streams differ);
    the episode Log (the reference GPU env's 13 fields, replayed from the
    oracle's rewards and diagnostics) bit-equal, the puf_live_log totals equal;
  - the reference core's fixture (obs / state SHA-256, reward bits) on the
    7-room plan and on a plan at building_train_1's size (205,434 cells);
  - default field mode: state within the per-step bar (1e-9 relative),
    observations within float32 quantization of the physics fields, rewards
    within 2 float32 ulps;
  - a vec mixing RC layouts and a field scenario: every env against its
    oracle twin (RC envs at the RC tolerances);
  - stochastic convection on (the shipped buildings' p = 0.1 within distance
    2, and p = 0.6 in a room of 45,384 cells, whose swap pairs outgrow the
    plan kernel's LDS): the same bit-identity in exact mode, the tolerances in
    default mode, and the reference core's fixture at 205,434 cells.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import pytest

import pyoracle as po

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from neurips2026_smart_building_challenge_amd import env as E  # noqa: E402
from neurips2026_smart_building_challenge_amd.scenario import fdm as F  # noqa: E402
from neurips2026_smart_building_challenge_amd.scenario import generate as G  # noqa: E402
from neurips2026_smart_building_challenge_amd.scenario.sbb import read_sbb  # noqa: E402

GOLDEN = Path(__file__).resolve().parent / "golden"
SEED = 777
STATE_RTOL = 1e-9
SMALL = dict(rows=120, cols=90, rooms=7, margin=6, seed=3)


def say(msg: str) -> None:
    print(f"[field env] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    yield
    torch.cuda.synchronize()


SHIPPED_CONV = (0.1, 2, 5)


def field_blob(tmp: Path, field: dict, ahus: int, clim: int, table_steps: int = G.EPISODE_STEPS + 256,
               conv=None) -> Path:
    spec = G.FieldEnvSpec(F.FdmSpec(**field), ahus)
    cv = None if conv is None else G.ConvSpec(*conv)
    data = G.field_env_writer(spec, G.climates()[clim], table_steps, 17321, cv).tobytes()
    p = tmp / f"{spec.name}__c{clim}{'' if cv is None else '__' + cv.tag}.sbb"
    p.write_bytes(data)
    return p


@pytest.fixture(scope="module")
def small_blob(tmp_path_factory):
    return field_blob(tmp_path_factory.mktemp("field_small"), SMALL, 2, 1)


@pytest.fixture(scope="module")
def small_conv_blob(tmp_path_factory):
    return field_blob(tmp_path_factory.mktemp("field_small_conv"), SMALL, 2, 1, conv=SHIPPED_CONV)


def host(t) -> np.ndarray:
    return t.detach().cpu().numpy()


class Twin:
    def __init__(self, vec: E.VecEnv, i: int, max_steps: int):
        path, start, seed = vec.meta(i)
        self.i = i
        self.cpu = po.CpuEnv("oracle", path, seed, start=start, max_steps=max_steps)
        d = read_sbb(path)
        self.obs_len = int(d["n_dev"][0] + d["n_aux"][0])
        n_dev = self.obs_len - int(d["n_aux"][0])
        kind, oid = d["f_dev_kind"], d["f_obs_id"]
        self.exact = np.ones(self.obs_len, bool)
        for f in range(n_dev):
            if (kind[f] == 1 and oid[f] == 5) or (kind[f] == 0 and oid[f] in (2, 5, 6)):
                self.exact[f] = False   # sensed zone temperatures and AHU flows come from the field
        self.mean = np.zeros(self.obs_len)
        self.sd = np.ones(self.obs_len)
        self.mean[:n_dev] = d["f_norm_mean"]
        self.sd[:n_dev] = np.sqrt(np.maximum(d["f_norm_var"], 0.0))

        # the reference GPU env's episode log, replayed from the oracle's steps
        self.glog = po.GpuEnvLog()
        self.steps = 0

    def step(self, s):
        out = self.cpu.step(po.action_row(SEED, self.i, s, self.cpu.n_cont, self.cpu.n_disc))
        self.steps += 1
        self.glog.step(out[1], self.cpu.parts(), self.steps, bool(out[2]), False)
        if out[2]:
            self.steps = 0
        return out


def obs_close(g: np.ndarray, tw: Twin, c: np.ndarray, where: str):
    n = tw.obs_len
    assert np.all(g[n:] == 0.0), f"{where}: padding not zero"
    ex = tw.exact
    bad = np.nonzero(g[:n][ex].view(np.uint32) != c[:n][ex].view(np.uint32))[0]
    assert bad.size == 0, f"{where}: exact obs fields differ at {np.nonzero(ex)[0][bad][:8]}"
    raw = c[:n].astype(np.float64) * tw.sd + tw.mean
    tol = (np.spacing(np.abs(raw).astype(np.float32)).astype(np.float64) / np.where(tw.sd > 0, tw.sd, 1.0)
           + 2 * np.spacing(np.abs(c[:n])).astype(np.float64) + 1e-30)
    err = np.abs(g[:n].astype(np.float64) - c[:n].astype(np.float64))
    assert np.all(err[~ex] <= tol[~ex]), f"{where}: obs beyond float32 quantization"


def run_against_oracle(vec, twins, steps, exact: bool, tag: str):
    vec.reset()
    for tw in twins:
        ob = tw.cpu.reset()
        g = host(vec.obs[tw.i])
        assert np.array_equal(g[:tw.obs_len], ob[:tw.obs_len]) and np.all(g[tw.obs_len:] == 0.0), f"{tag} reset obs"
    done_seen = 0
    for s in range(steps):
        vec.gen_actions(SEED, s)
        vec.step()
        torch.cuda.synchronize()
        obs, rew, term = host(vec.obs), host(vec.rewards), host(vec.terminals)
        for tw in twins:
            ob, r, t, _ = tw.step(s)
            where = f"{tag} env {tw.i} step {s}"
            assert term[tw.i] == t, where
            done_seen += int(t)
            cs = tw.cpu.state()
            gs = vec.state(tw.i)[:cs.size]
            if exact:
                assert np.array_equal(obs[tw.i][:tw.obs_len], ob[:tw.obs_len]), f"{where}: obs"
                assert np.float32(rew[tw.i]) == np.float32(r), f"{where}: reward {rew[tw.i]} vs {r}"
                assert np.array_equal(gs, cs), f"{where}: state differs at {np.nonzero(gs != cs)[0][:8]}"
            else:
                obs_close(obs[tw.i], tw, ob, where)
                assert abs(float(rew[tw.i]) - r) <= 2 * np.spacing(np.float32(abs(r))) + 1e-12, f"{where}: reward"
                err = np.abs(gs - cs) / np.maximum(np.abs(cs), 1e-6)
                assert err.max() <= STATE_RTOL, f"{where}: state rel err {err.max():.3e} at {err.argmax()}"
    return done_seen


@pytest.mark.parametrize("conv", [False, True])
def test_gpu_field_env_exact_matches_oracle(small_blob, small_conv_blob, conv):
    blob = small_conv_blob if conv else small_blob
    say(f"3 envs, 7-room FDM plan{' with convection' if conv else ''}, exact field mode, 60 steps (auto-reset at 40)")
    vec = E.VecEnv(3, blob=str(blob), max_steps=40, field_exact=1)
    twins = [Twin(vec, i, 40) for i in range(3)]
    assert len({tw.cpu.n_cont for tw in twins}) == 1
    done = run_against_oracle(vec, twins, 60, True, "exact")
    assert done == 3, "every env ended its first episode at step 40"
    for tw in twins:
        # exact mode: the env's diagnostics are the oracle's to the bit, so is the Log
        got = vec.log(tw.i)
        want = {k: float(v) for k, v in tw.glog.log.items()}
        assert got == want, (tw.i, got, want)
        assert got["n"] == 1.0 and got["episode_length"] == 40.0
    live = vec.live_log()
    assert live["env_steps"] == 180.0 and live["episodes"] == 3.0
    vec.close()


@pytest.mark.parametrize("conv", [False, True])
def test_gpu_field_env_default_mode(small_blob, small_conv_blob, conv):
    say(f"3 envs, 7-room FDM plan{' with convection' if conv else ''}, default field mode, 50 steps")
    vec = E.VecEnv(3, blob=str(small_conv_blob if conv else small_blob), max_steps=30)
    twins = [Twin(vec, i, 30) for i in range(3)]
    run_against_oracle(vec, twins, 50, False, "default")
    vec.close()


@pytest.mark.parametrize("name", ["field_small", "field_train1_size", "field_small_conv", "field_train1_conv"])
def test_gpu_field_env_reference_fixture(name, tmp_path):
    fx = json.loads((GOLDEN / "field_env.json").read_text())
    case = fx["cases"][name]
    path = field_blob(tmp_path, case["field"], case["ahus"], case["climate"], fx["table_steps"], case.get("conv"))
    assert hashlib.sha256(path.read_bytes()).hexdigest() == case["blob_sha256"], "stale fixture"
    say(f"{name}: reference fixture, {case['steps']} steps, exact field mode")
    vec = E.VecEnv(1, blob=str(path), max_steps=case["max_steps"], field_exact=1)
    assert vec.meta(0)[1] == case["start"] and vec.meta(0)[2] == case["occ_seed"]
    vec.reset()
    n = read_sbb(path)["n_dev"][0] + read_sbb(path)["n_aux"][0]

    def dg(a):
        return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()

    torch.cuda.synchronize()
    assert dg(host(vec.obs[0])[:n]) == case["obs_sha"][0]
    assert dg(vec.state(0)[:-2]) == case["state_sha"][0]
    for s in range(case["steps"]):
        vec.gen_actions(fx["action_seed"], s)
        vec.step()
        torch.cuda.synchronize()
        assert dg(host(vec.obs[0])[:n]) == case["obs_sha"][s + 1], (name, s, "obs")
        assert dg(vec.state(0)[:-2]) == case["state_sha"][s + 1], (name, s, "state")
        assert int(np.float32(host(vec.rewards)[0]).view(np.uint32)) == case["reward_bits"][s], (name, s, "reward")
        assert float(host(vec.terminals)[0]) == case["terminal"][s], (name, s, "terminal")
    vec.close()


def test_gpu_field_env_mixed_with_rc(small_blob, tmp_path):
    """Two RC layouts and one field scenario in one vec (two envs each)."""
    d = tmp_path / "mixed"
    d.mkdir()
    for z, a in ((41, 1), (49, 2)):
        spec = G.LayoutSpec(z, a)
        clim = G.ClimateSpec(12.0, 8.0, seed=502)
        (d / f"{spec.name}__{clim.name}.sbb").write_bytes(
            G.scenario_writer(spec, clim, G.EPISODE_STEPS + 256, 17321).tobytes())
    (d / small_blob.name).write_bytes(small_blob.read_bytes())
    say("mixed vec: 2 RC layouts + 1 field scenario, 6 envs, 25 steps")
    vec = E.VecEnv(6, blob_dir=str(d), groups=3, max_steps=200)
    twins = [Twin(vec, i, 200) for i in range(6)]
    fields = [i for i in range(6) if "fdm_" in vec.meta(i)[0]]
    assert len(fields) == 2
    vec.reset()
    for tw in twins:
        tw.cpu.reset()
    for s in range(25):
        vec.gen_actions(SEED, s)
        vec.step()
        torch.cuda.synchronize()
        obs, rew = host(vec.obs), host(vec.rewards)
        for tw in twins:
            ob, r, t, _ = tw.step(s)
            where = f"mixed env {tw.i} step {s}"
            obs_close(obs[tw.i], tw, ob, where)
            cs = tw.cpu.state()
            gs = vec.state(tw.i)[:cs.size]
            fin = ~np.isnan(gs)
            err = np.abs(gs[fin] - cs[fin]) / np.maximum(np.abs(cs[fin]), 1e-6)
            assert err.max() <= STATE_RTOL, f"{where}: state rel err {err.max():.3e}"
            assert abs(float(rew[tw.i]) - r) <= 4 * np.spacing(np.float32(abs(r))) + 1e-12, where
    vec.close()


def test_gpu_field_env_conv_big_room(tmp_path):
    """Two rooms, the larger of 45,384 cells, with p = 0.6: about 27,000 swap
    pairs a step there, more than the plan kernel holds in LDS beside the
    room's permutation (the rest go to its HBM overflow), and room-local
    indices in the upper half of the 16-bit range. Exact mode, bit-identical
    to the oracle every step."""
    field = dict(rows=310, cols=260, rooms=2, margin=6, seed=4)
    blob = field_blob(tmp_path, field, 2, 2, conv=(0.6, 2, 9))
    assert int(np.diff(read_sbb(blob)["conv_room_offsets"]).max()) == 45384
    say("3 envs, rooms of 45,384 and 26,108 cells, convection p = 0.6, exact field mode, 6 steps")
    vec = E.VecEnv(3, blob=str(blob), max_steps=100, field_exact=1)
    twins = [Twin(vec, i, 100) for i in range(3)]
    run_against_oracle(vec, twins, 6, True, "big room")
    vec.close()


def test_gpu_field_env_default_mode_full_size(tmp_path):
    """building_train_1's size (205,434 cells) with the shipped buildings'
    convection, default field mode, 300 envs (the field group then runs two
    envs per block), episodes of 3 steps: four envs against their oracle twins
    every step through two auto-resets: state within 1e-9, observations within
    float32 quantisation of the physics fields, rewards within 2 float32 ulps."""
    blob = field_blob(tmp_path, {}, 3, 3, conv=SHIPPED_CONV)
    G = 300
    say(f"{G} envs at 205,434 cells with convection, default field mode, 7 steps (resets after 3 and 6)")
    vec = E.VecEnv(G, blob=str(blob), max_steps=3)
    picks = [0, 1, 150, G - 1]
    twins = [Twin(vec, i, 3) for i in picks]
    done = run_against_oracle(vec, twins, 7, False, "full size")
    assert done == 2 * len(picks)
    vec.close()


LARGEST = dict(rows=1622, cols=653, rooms=82, seed=3)   # building_30025__singapore_5's grid and rooms


@pytest.fixture(scope="module")
def largest_blob(tmp_path_factory):
    p = field_blob(tmp_path_factory.mktemp("field_largest"), LARGEST, 4, 3, table_steps=64, conv=SHIPPED_CONV)
    yield p
    p.unlink()


@pytest.mark.parametrize("exact", [True, False])
def test_gpu_field_env_largest_shipped_size(largest_blob, exact):
    """The largest shipped building's size (1,059,166 cells, 926,266 solved,
    82 rooms, 4 AHUs) with the shipped convection (p 0.1, distance 2): two envs
    against their oracle twins through an auto-reset, bit-identical in exact
    field mode, within the per-step bars in the default one."""
    say(f"2 envs at 1,059,166 cells with convection, {'exact' if exact else 'default'} field mode, 4 steps")
    vec = E.VecEnv(2, blob=str(largest_blob), max_steps=3, field_exact=1 if exact else 0)
    twins = [Twin(vec, i, 3) for i in range(2)]
    done = run_against_oracle(vec, twins, 4, exact, "largest")
    assert done == 2
    vec.close()


def test_gpu_cont_big_build():
    """The SB_CONT_BIG build (320 continuous heads) steps a field scenario with
    260 continuous actions beside an RC layout, against the oracle built the
    same way, and runs the shared policy over 336-wide action rows; the build
    is chosen at import, so tests/cont_big_check.py runs in a child process."""
    import os
    import subprocess
    import sys

    say("SB_CONT_BIG build: field scenario with 260 continuous actions + RC layout, child process")
    r = subprocess.run([sys.executable, "-u", str(Path(__file__).resolve().parent / "cont_big_check.py")],
                       env={**os.environ, "SBENV_CONT_BIG": "1"}, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0 and "cont_big ok" in r.stdout, (r.stdout[-3000:], r.stderr[-3000:])
