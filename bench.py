"""Benchmark of the MI355X env step: env-steps/s at 960 mixed envs (fp64 physics).

    python bench.py [--steps K] [--warmup W] [--config 1] [--gpus 1] [--no-cpu] [--conv P]

Workload (BASELINE config index 1): 960 envs over 30 seeded synthetic scenarios
(6 layouts of 41..81 zones x 5 climates, 32 envs each), Beta(2,2) actions from
the on-device counter RNG, fp64 physics. The action rows of all K timed steps
are drawn before the timed region (sbx_gen_actions, the policy stand-in) and
stay resident in HBM; one timed step = one env step over all envs reading its
own rows (sbx_step_actions, puf_step with a per-step action pointer), as the
reference's bench feeds recorded action traces to its step. The JSON also
reports the generator + step pair launched in turn (generator_and_step_us).
K defaults to a full 8,640-step episode. Config 4 times the rollout: policy
forward + Beta sampling, then puf_step, each step. Configs 0-3 are timed a
second time with the per-env sparse LU as the field solver (the "lu" record).
Config 1 also times the building-scale field step (the "fdm" record, see
fdm_leg; --fdm-only runs just that) and whole env steps of FDM-scale
scenarios through the same ABI (the "field_env" record, see field_env_leg).

roofline: algorithmic HBM bytes of one puf_step (per env: the persistent state
read and written -- T, per-VAV and per-AHU state, plant scalars, occupancy,
interior mass -- the action row read, the observation prefix, reward and
terminal written; the shared per-layout/per-scenario tables are not counted)
divided by the step kernel's mean duration: the timed region itself (it launches only step
kernels, back to back on the bound stream) for configs 0-3; for config 4, HIP
event pairs recorded around every 16th step-kernel launch (bracketing every
launch would add queue markers that slow the loop itself). traffic: HBM bytes per launch
from rocprofv3 FETCH_SIZE / WRITE_SIZE passes, scaled by the same counters on a
plain copy of known size (--calibrate-copy), when profiles/ holds them.

cpu_baseline: the reference csim core (oracle/_ref, compiled from the
reference sources) or, where it was not built, this repo's C restatement,
stepping the same 960 envs on the host's cores (whole envs per thread) for a
bounded number of steps.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "env-steps/sec at 960 mixed envs (fp64 physics); % of HBM roofline"
HBM_PEAK_GBS = 8000.0
SEED = 20260601
TIMER_PERIOD = 16   # every 16th step-kernel launch of the timed region is bracketed by HIP events
CPU_FIELD_BUDGET_S = 10.0   # wall clock of the building-scale CPU baselines
SHIPPED_CONV = (0.1, 2, 5)  # stochastic convection of every shipped building (data/blob_meta/*.json "conv")


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def scenario_dir(config: int, conv: float = 0.0) -> Path:
    """The config's blobs; conv > 0 turns stochastic convection on in every blob
    (probability conv per room cell and step, candidates within 2 columns)."""
    from neurips2026_smart_building_challenge_amd.scenario import generate as G

    cv = G.ConvSpec(conv, 2, 9001) if conv > 0 else None
    d = Path(tempfile.gettempdir()) / (f"sbenv_bench_cfg{config}" + (f"_{cv.tag}" if cv else ""))
    G.write_config(config, d, conv=cv)
    return d


def measured_traffic(config: int):
    p = ROOT / "profiles" / f"step_kernel_traffic_cfg{config}.json"
    if p.exists():
        try:
            return float(json.loads(p.read_text())["hbm_bytes_per_launch"])
        except Exception:
            return None
    return None


def cpu_baseline(blob_dir: Path, n_envs: int, groups: int, target_s: float, threads: int) -> dict:
    sys.path.insert(0, str(ROOT / "oracle"))
    import pyoracle as po
    from neurips2026_smart_building_challenge_amd.scenario import generate as G
    from neurips2026_smart_building_challenge_amd.scenario.sbb import read_sbb

    kind = "ref" if po.ref_available() else "oracle"
    paths = sorted(blob_dir.glob("*.sbb"))
    # same assignment as the GPU vec: round-robin over buildings, n/G envs per scenario
    blds = []
    for p in paths:
        b = p.name.split("__")[0]
        if b not in blds:
            blds.append(b)
    ordered, used = [], set()
    while len(ordered) < len(paths):
        for b in blds:
            for p in paths:
                if p not in used and p.name.split("__")[0] == b:
                    ordered.append(p)
                    used.add(p)
                    break
    ordered = ordered[:groups]
    envs, ids = [], []
    for g, p in enumerate(ordered):
        seed0 = int(read_sbb(p)["occ_seed"][0])
        cnt = n_envs // groups + (1 if g < n_envs % groups else 0)
        for j in range(cnt):
            e = po.CpuEnv(kind, p, seed0 + j, start=0, max_steps=G.EPISODE_STEPS)
            e.reset()
            envs.append(e)
            ids.append(len(ids))
    secs, _ = po.run_batch(envs, ids, 4, SEED, threads)          # calibration
    per_step = secs / 4
    steps = max(4, min(G.EPISODE_STEPS, int(target_s / max(per_step, 1e-9))))
    secs, _ = po.run_batch(envs, ids, steps, SEED + 1, threads)
    # one core: every 8th env (all 30 scenarios stay represented), about a third of the time
    sub_envs, sub = envs[::8], ids[::8]
    s1, _ = po.run_batch(sub_envs, sub, 2, SEED + 2, 1)
    steps1 = max(2, int(target_s / 3 / max(s1 / 2, 1e-9)))
    s1, _ = po.run_batch(sub_envs, sub, steps1, SEED + 3, 1)
    for e in envs:
        e.close()
    return {"value": n_envs * steps / secs, "unit": "env-steps/s", "cores": threads,
            "kind": "reference" if kind == "ref" else "port",
            "value_single_core": len(sub) * steps1 / s1,
            "sample": f"{n_envs} envs of the same workload x {steps} steps ({secs:.1f} s) on {threads} threads "
                      f"(whole envs per thread); single core: {len(sub)} of the envs x {steps1} steps "
                      f"({s1:.1f} s); {'reference csim compiled from its sources' if kind == 'ref' else 'C restatement of csim'}"}


def calibrate_copy() -> int:
    """A plain device-to-device copy of known size, for scaling the HBM counters."""
    import torch

    n = 256 << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").random_(0, 255)
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "copies": 10}), flush=True)
    return 0


def timed_cpu_steps(handles, step, budget_s: float) -> tuple[float, int, float]:
    """Steps every handle once untimed (each on its own thread), then keeps
    stepping all of them in rounds until `budget_s` of wall clock has passed.
    Returns (env-steps/s, rounds timed, seconds timed)."""
    from concurrent.futures import ThreadPoolExecutor

    with ThreadPoolExecutor(len(handles)) as ex:
        list(ex.map(step, handles))
        rounds, t0 = 0, time.time()
        while True:
            list(ex.map(step, handles))
            rounds += 1
            dt = time.time() - t0
            if dt >= budget_s:
                break
    return rounds * len(handles) / dt, rounds, dt


def fdm_leg(envs: int, steps: int, cpu: bool, cpu_threads: int) -> dict:
    """The building-scale field step (sbx_fdm_step, the reference's
    sb_fdm_step_batch) on a seeded FDM plan at building_train_1's size (606 x
    339 cells, 39 rooms, SuperLU factors with the reference baker's options):
    `envs` envs in one group, inputs resident in HBM (the seeded step inputs of
    8 envs repeated), `steps` timed steps after one untimed step. cpu: the
    reference core's sb_fdm_step_batch (oracle/_ref; this repo's restatement
    where that is not built) on `cpu_threads` threads, one env each, one
    untimed step, then timed steps for CPU_FIELD_BUDGET_S."""
    import numpy as np
    import torch

    from neurips2026_smart_building_challenge_amd.fdm import FieldGroup
    from neurips2026_smart_building_challenge_amd.scenario import fdm as F

    spec = F.FdmSpec()
    plan = F.make_plan(spec)
    td = Path(tempfile.mkdtemp(prefix="sb_fdm_"))
    path = td / f"{spec.name}.sbb"
    path.write_bytes(F.fdm_writer(plan).tobytes())
    f = FieldGroup(path, envs)
    inf = f.info
    inp = F.step_inputs(plan, 8, SEED, 0)
    rep = lambda a: np.ascontiguousarray(np.concatenate([a] * (envs // a.shape[0] + 1))[:envs])
    dev = [torch.from_numpy(x).cuda() for x in (rep(inp["input_q"]), rep(inp["ambient"]), rep(inp["h"]),
                                                  rep(inp["air_g"]), rep(inp["air_T"]))]
    f.step(*dev)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        f.step(*dev)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    rec = {"workload": f"FDM field step, {plan.n_cvs} cells ({plan.n} solved), {plan.k} rooms, SuperLU factors "
                       f"({inf.nnz_l} + {inf.nnz_u} off-diagonal, {inf.levels_l}/{inf.levels_u} levels), "
                       f"{envs} envs, air side on",
           "n_envs": envs, "steps": steps, "ms_per_step": ms, "value": envs / (ms / 1e3), "unit": "env-steps/s",
           "mode": "default (LDS runs of the narrow levels, chunked levels, air-side correction from the applied columns' responses)",
           "lds_run_rows": [inf.tail_rows_l, inf.tail_rows_u], "lds_run_levels": [inf.tail_levels_l, inf.tail_levels_u],
           "algorithmic_bytes": inf.bytes_per_step,
           "achieved_gbs": inf.bytes_per_step / (ms / 1e3) / 1e9}
    f.close()
    log(f"fdm field step: {ms:.2f} ms/step at {envs} envs, {rec['value']:.4g} env-steps/s")
    if cpu:
        sys.path.insert(0, str(ROOT / "oracle"))
        import pyoracle as po

        kind = "ref" if po.ref_available() else "oracle"
        hs = [po.Fdm(kind, path, 1) for _ in range(cpu_threads)]
        one = {k: (v[:1] if np.ndim(v) else v) for k, v in inp.items()}
        rate, rounds, dt = timed_cpu_steps(hs, lambda h: h.step(one), CPU_FIELD_BUDGET_S)
        rec["cpu_baseline"] = {"value": rate, "unit": "env-steps/s", "cores": cpu_threads,
                               "kind": "reference" if kind == "ref" else "port",
                               "sample": f"{cpu_threads} envs, one per thread, one untimed step each, then "
                                         f"{rounds} timed steps each ({dt:.1f} s)"}
        log(f"fdm cpu baseline: {rec['cpu_baseline']['value']:.4g} env-steps/s on {cpu_threads} threads ({kind})")
        for h in hs:
            h.close()
    return rec


def with_more_envs(leg, envs: int, cpu: bool, cpu_threads: int, more=()) -> dict:
    """A building-scale record at `envs` envs, with the same leg timed (3
    steps, no CPU baseline) at each of `more` envs beside it: the reference's
    published GPU figures are quoted at 256 and 512 envs."""
    rec = leg(envs, 5, cpu, cpu_threads)
    rec["more_envs"] = []
    for m in more:
        if m != envs:
            r = leg(m, 3, False, 1)
            rec["more_envs"].append({k: r[k] for k in ("n_envs", "steps", "ms_per_step", "value")})
    return rec


def field_env_leg(envs: int, steps: int, cpu: bool, cpu_threads: int) -> dict:
    """Whole env steps (puf_step on pre-drawn resident action rows) of an
    FDM-scale scenario: the field of building_train_1's size (606 x 339 cells,
    39 rooms; fdm.FdmSpec()) with one VAV per room and 3 AHUs
    (generate.field_env_writer), `envs` envs, `steps` timed steps after one
    untimed step; stochastic convection on as in every shipped building (p =
    0.1 per room cell and step, candidates within distance 2). cpu: the
    reference core's env (oracle/_ref; this repo's restatement where that is
    not built) on `cpu_threads` threads, one env each, one untimed step, then
    timed steps for CPU_FIELD_BUDGET_S."""
    import torch

    from neurips2026_smart_building_challenge_amd import env as E
    from neurips2026_smart_building_challenge_amd.scenario import fdm as F
    from neurips2026_smart_building_challenge_amd.scenario import generate as G

    spec = G.FieldEnvSpec(F.FdmSpec(), 3)
    td = Path(tempfile.mkdtemp(prefix="sb_field_env_"))
    path = td / f"{spec.name}.sbb"
    path.write_bytes(G.field_env_writer(spec, G.climates()[2], G.EPISODE_STEPS + 256, 17321,
                                        G.ConvSpec(*SHIPPED_CONV)).tobytes())
    vec = E.VecEnv(envs, blob=str(path))
    info = vec.info()
    vec.reset()
    rows = torch.empty((steps + 1, envs, 272), dtype=torch.float32, device="cuda")
    for s in range(steps + 1):
        vec.gen_actions(SEED, s)
        rows[s].copy_(vec.actions)
    vec.step_actions(rows[0])
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for s in range(steps):
        vec.step_actions(rows[s + 1])
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    rec = {"workload": f"FDM-scale env scenario: {spec.field.rows} x {spec.field.cols} cells, {spec.field.rooms} rooms "
                       f"(one VAV each), {spec.ahus} AHUs, stochastic convection p = {SHIPPED_CONV[0]} within "
                       f"distance {SHIPPED_CONV[1]} (every shipped building's setting); {envs} envs through puf_step",
           "n_envs": envs, "steps": steps, "ms_per_step": ms, "value": envs / (ms / 1e3), "unit": "env-steps/s",
           "algorithmic_bytes": info.bytes_per_step, "achieved_gbs": info.bytes_per_step / (ms / 1e3) / 1e9}
    vec.close()
    log(f"field env step: {ms:.2f} ms/step at {envs} envs, {rec['value']:.4g} env-steps/s")
    if cpu:
        sys.path.insert(0, str(ROOT / "oracle"))
        import pyoracle as po

        kind = "ref" if po.ref_available() else "oracle"
        es = [po.CpuEnv(kind, path, 17321 + j) for j in range(cpu_threads)]
        for e in es:
            e.reset()
        row = po.action_row(SEED, 0, 0, es[0].n_cont, es[0].n_disc)
        rate, rounds, dt = timed_cpu_steps(es, lambda e: e.step(row), CPU_FIELD_BUDGET_S)
        rec["cpu_baseline"] = {"value": rate, "unit": "env-steps/s", "cores": cpu_threads,
                               "kind": "reference" if kind == "ref" else "port",
                               "sample": f"{cpu_threads} envs, one per thread, one untimed step each, then "
                                         f"{rounds} timed steps each ({dt:.1f} s), convection on"}
        log(f"field env cpu baseline: {rec['cpu_baseline']['value']:.4g} env-steps/s on {cpu_threads} threads ({kind})")
        for e in es:
            e.close()
    return rec


def config_leg(config: int, steps: int, warmup: int) -> dict:
    """One other BASELINE config (index 0, 2, 3 or 4) timed the headline's way:
    action rows of every timed step drawn before the timed region (config 4:
    the shared-policy forward + Beta sampling, then puf_step, each step), the
    env step's mean duration over the timed region. Reported beside the
    headline so every config is timed by the same run."""
    import torch

    from neurips2026_smart_building_challenge_amd import env as E
    from neurips2026_smart_building_challenge_amd.scenario import generate as G

    scen, n_envs, offsets = G.config_scenarios(config)
    groups = len(scen)
    blob_dir = scenario_dir(config)
    vec = E.VecEnv(n_envs, blob_dir=str(blob_dir), groups=groups, start_offsets=int(offsets))
    info = vec.info()
    rollout = config == 4
    if rollout:
        vec.policy_bind(E.policy_weights(SEED))
    vec.reset()
    for s in range(warmup):
        if rollout:
            vec.policy_act(SEED, s)
        else:
            vec.gen_actions(SEED, s)
        vec.step()
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    bank = None
    if not rollout:
        bank = torch.empty((steps, n_envs, E.SB_ACT), dtype=torch.float32, device="cuda")
        for s in range(steps):
            vec.gen_actions(SEED, warmup + s)
            bank[s].copy_(vec.actions)
    torch.cuda.synchronize()
    ev0.record(stream)
    for s in range(steps):
        if rollout:
            vec.policy_act(SEED, warmup + s)
            vec.step()
        else:
            vec.step_actions(bank[s])
    ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1)
    vec.close()
    del bank
    us = ms / steps * 1e3
    value = n_envs * steps / (ms / 1e3)
    ach = info.bytes_per_step / (us * 1e-6) / 1e9
    rec = {"config": config, "n_envs": n_envs, "scenarios": groups, "steps": steps, "warmup": warmup,
           "workload": f"BASELINE config {config}: {n_envs} envs, {groups} scenarios"
                       + (", desynchronised starts" if offsets else "")
                       + (", shared-policy MLP + Beta sampling then puf_step per step" if rollout
                          else ", Beta(2,2) action rows resident, puf_step per step"),
           "ms_per_step": ms / steps, "value": value, "unit": "env-steps/s",
           "roofline": None if rollout else {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                              "frac": ach / HBM_PEAK_GBS, "kernel_us": us,
                                              "algorithmic_bytes": info.bytes_per_step}}
    log(f"config {config}: {us:.1f} us/step over {steps} steps, {value:.4g} env-steps/s")
    return rec


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=8640)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--config", type=int, default=1)
    ap.add_argument("--kernel-iters", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-lu", action="store_true", help="skip the second timing under the LU solver")
    ap.add_argument("--solver", default="auto", choices=["auto", "relax", "point", "lu"])
    ap.add_argument("--conv", type=float, default=0.0,
                    help="stochastic convection on with this swap probability (not a BASELINE config)")
    ap.add_argument("--fdm-envs", type=int, default=256, help="envs of the building-scale field-step record (0: skip)")
    ap.add_argument("--fdm-only", action="store_true", help="only the building-scale field-step record")
    ap.add_argument("--more-envs", type=str, default="512",
                    help="comma-separated env counts the building-scale records are also timed at (0: none)")
    ap.add_argument("--field-env-envs", type=int, default=256,
                    help="envs of the FDM-scale env-scenario record (0: skip)")
    ap.add_argument("--field-env-only", action="store_true", help="only the FDM-scale env-scenario record")
    ap.add_argument("--other-configs", type=str, default="0,2,3,4",
                    help="comma-separated other BASELINE configs timed after the headline (config 1 runs only); "
                         "'' for none")
    ap.add_argument("--other-steps", type=int, default=200,
                    help="timed steps of each other config (at most --steps)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain device copy of 256 MiB 10 times (counter calibration)")
    args = ap.parse_args()
    if args.calibrate_copy:
        return calibrate_copy()
    if args.gpus != 1:
        log("bench.py measures one GPU: the env step has no cross-GPU exchange and this build runs "
            "on a single MI355X; --gpus above 1 is not supported")
        return 2

    import torch

    from neurips2026_smart_building_challenge_amd import env as E
    from neurips2026_smart_building_challenge_amd.scenario import generate as G

    more = tuple(m for m in (int(x) for x in args.more_envs.split(",") if x.strip()) if m > 0)
    if args.fdm_only:
        visible = len(os.sched_getaffinity(0))
        print(json.dumps(with_more_envs(fdm_leg, max(1, args.fdm_envs), not args.no_cpu, min(16, visible), more)),
              flush=True)
        return 0
    if args.field_env_only:
        visible = len(os.sched_getaffinity(0))
        print(json.dumps(with_more_envs(field_env_leg, max(1, args.field_env_envs), not args.no_cpu,
                                        min(16, visible), more)), flush=True)
        return 0
    scen, n_envs, offsets = G.config_scenarios(args.config)
    groups = len(scen)
    t0 = time.time()
    blob_dir = scenario_dir(args.config, args.conv)
    log(f"scenarios ready in {time.time() - t0:.1f}s: {blob_dir}")
    vec = E.VecEnv(n_envs, blob_dir=str(blob_dir), groups=groups, start_offsets=int(offsets), solver=args.solver)
    info = vec.info()
    rollout = args.config == 4
    if rollout:
        # the shared-policy MLP (fp32 MFMA) + Beta sampling makes every action row
        vec.policy_bind(E.policy_weights(SEED))

        def actions(s):
            vec.policy_act(SEED, s)
    else:
        def actions(s):
            vec.gen_actions(SEED, s)
    vec.reset()
    for s in range(args.warmup):
        actions(s)
        vec.step()
    torch.cuda.synchronize()
    log(f"warmup done ({args.warmup} steps)")
    bank = None
    if not rollout:
        # the Beta(2,2) action rows of every timed step, drawn before the timed
        # region so the timed steps find their inputs resident in HBM
        bank = torch.empty((args.steps, n_envs, E.SB_ACT), dtype=torch.float32, device="cuda")
        for s in range(args.steps):
            vec.gen_actions(SEED, args.warmup + s)
            bank[s].copy_(vec.actions)
        torch.cuda.synchronize()
        log(f"action rows of {args.steps} steps drawn ({bank.numel() * 4 / 1e9:.2f} GB resident)")
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    if rollout:
        vec.kernel_timer(TIMER_PERIOD)   # the step kernel's own events, every 16th launch
    ev0.record(stream)
    if rollout:
        for s in range(args.steps):
            actions(args.warmup + s)
            vec.step()
    else:
        for s in range(args.steps):
            vec.step_actions(bank[s])
    ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1)
    lu = None
    if not rollout and args.solver == "auto" and not args.no_lu:
        # the north star's per-env sparse LU (numeric refactorization + both
        # triangular solves every step) on the same envs and action rows
        lvec = E.VecEnv(n_envs, blob_dir=str(blob_dir), groups=groups, start_offsets=int(offsets), solver="lu")
        lvec.reset()
        for s in range(args.warmup):
            lvec.gen_actions(SEED, s)
            lvec.step()
        torch.cuda.synchronize()
        ev0.record(stream)
        for s in range(args.steps):
            lvec.step_actions(bank[s])
        ev1.record(stream)
        torch.cuda.synchronize()
        lms = ev0.elapsed_time(ev1)
        linfo = lvec.info()
        l_us = lms / args.steps * 1e3
        l_ach = linfo.bytes_per_step / (l_us * 1e-6) / 1e9
        lu = {"solver": "lu", "ms_per_step": lms / args.steps, "value": n_envs * args.steps / (lms / 1e3),
              "unit": "env-steps/s", "steps": args.steps,
              "roofline": {"bound": "hbm", "achieved": l_ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": l_ach / HBM_PEAK_GBS, "kernel_us": l_us,
                           "algorithmic_bytes": linfo.bytes_per_step},
              "solve_flops_per_step": linfo.flops_per_step}
        log(f"LU solver: {l_us:.1f} us/step, {lu['value']:.4g} env-steps/s")
        lvec.close()
    if rollout:
        k_us, k_n = vec.kernel_timer(0)
        k_src = "HIP event pairs around every 16th step-kernel launch of the timed region"
    else:
        # the timed region holds only step-kernel launches: their mean duration
        k_us, k_n = ms / args.steps * 1e3, args.steps
        k_src = "HIP events around the timed region of back-to-back step-kernel launches"
    gen_step_us = None
    if not rollout:
        # for reference: the generator kernel and the step launched in turn each step
        del bank
        m = min(args.steps, 1000)
        torch.cuda.synchronize()
        ev0.record(stream)
        for s in range(m):
            vec.gen_actions(SEED, args.warmup + args.steps + s)
            vec.step()
        ev1.record(stream)
        torch.cuda.synchronize()
        gen_step_us = ev0.elapsed_time(ev1) / m * 1e3
    ms_per_step = ms / args.steps
    value = n_envs * args.steps / (ms / 1e3)
    log(f"timed {args.steps} steps: {ms_per_step * 1e3:.1f} us/step, {value:.4g} env-steps/s")
    achieved = info.bytes_per_step / (k_us * 1e-6) / 1e9
    log(f"step kernel: {k_us:.1f} us/launch over {k_n} launches, {info.bytes_per_step / 1e6:.2f} MB "
        f"algorithmic -> {achieved:.1f} GB/s")
    b2b_us = vec.time_step(max(1, args.kernel_iters)) / max(1, args.kernel_iters) * 1e3
    solver = vec.solve_info(0)
    sweeps = [vec.solve_info(i)["sweeps"] for i in range(0, n_envs, max(1, n_envs // 64))]
    traffic = measured_traffic(args.config) if args.conv <= 0 else None
    phases = vec.phase_times()
    log("phase us (mean / max over workgroups): " +
        ", ".join(f"{k} {m:.1f}/{x:.1f}" for k, (m, x) in phases.items()))
    vec.close()

    cpu = None
    if not args.no_cpu:
        # every core the process may run on, up to the 16-core CPU share a
        # one-GPU box of this pool grants a job (a process pool must not exceed it)
        visible = len(os.sched_getaffinity(0))
        threads = min(16, visible)
        log(f"cpu baseline on {threads} threads ({visible} cores visible) ...")
        cpu = cpu_baseline(blob_dir, n_envs, groups, args.cpu_seconds, threads)
        cpu["cores_visible"] = visible
        log(f"cpu baseline: {cpu['value']:.4g} env-steps/s ({cpu['kind']})")

    fdm = field_env = None
    if args.fdm_envs > 0 and args.config == 1 and args.conv <= 0:
        fdm = with_more_envs(fdm_leg, args.fdm_envs, not args.no_cpu, min(16, len(os.sched_getaffinity(0))), more)
    if args.field_env_envs > 0 and args.config == 1 and args.conv <= 0:
        field_env = with_more_envs(field_env_leg, args.field_env_envs, not args.no_cpu,
                                   min(16, len(os.sched_getaffinity(0))), more)

    others = []
    if args.config == 1 and args.conv <= 0:
        for c in (int(x) for x in args.other_configs.split(",") if x.strip()):
            if c != 1:
                others.append(config_leg(c, max(1, min(args.steps, args.other_steps)), min(args.warmup, 20)))

    out = {
        "metric": METRIC, "value": value, "unit": "env-steps/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_per_step, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f64", "data": "synthetic",
        "config": {"workload": f"BASELINE config {args.config}: {n_envs} envs, {groups} scenarios "
                               f"({len({s[0].zones for s in scen})} layouts x {len({s[1].name for s in scen})} "
                               f"climates), "
                               + ("shared-policy MLP 1024-128-128-544 (fp32 MFMA) + Beta sampling per step, "
                                  if rollout else "Beta(2,2) actions, ")
                               + "fp64 physics" + (", desynchronised starts (seeded per-env calendar offsets)" if offsets else "")
                               + (f", stochastic convection p={args.conv}" if args.conv > 0 else ""),
                   "n_envs": n_envs, "scenarios": groups, "episode_steps": G.EPISODE_STEPS,
                   "solver": solver["solver"], "envs_per_workgroup": info.envs_per_block,
                   "block": info.block, "lds_bytes": info.lds_bytes},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "kernel_us": k_us, "kernel_launches_timed": k_n, "kernel_timing": k_src,
                     "back_to_back_us": b2b_us,
                     "generator_and_step_us": gen_step_us,
                     "algorithmic_bytes": info.bytes_per_step,
                     "record_bytes": info.record_bytes_per_step,
                     "relax_sweeps_mean": (sum(sweeps) / len(sweeps)) if solver["solver"] != "lu" else None,
                     "phase_us_mean": {k: round(m, 2) for k, (m, x) in phases.items()}},
        "cpu_baseline": cpu,
        "lu": lu,
        "fdm": fdm,
        "field_env": field_env,
        "other_configs": others,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
