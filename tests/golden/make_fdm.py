"""Writes tests/golden/fdm.json from the reference core's field model (the
compiled csim of oracle/_ref: sb_fdm_init and sb_fdm_step_batch,
complete_port/csim/sb_fdm.c:40-270), run only here, in the development
container:

    python tests/golden/make_fdm.py

Per case: the FDM plan spec (scenario/fdm.py regenerates the blob from it; its
SHA-256 is recorded so a generator change is caught), the group size, the
input seed, and after every step the SHA-256 of every env's field (T, n_cvs
f64) and interior mass (M, n_solved f64), plus a few cells' values for
readable failures. The inputs of step s are fdm.step_inputs(plan, G, seed, s).
"""
from __future__ import annotations

import hashlib
import json
import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))

from neurips2026_smart_building_challenge_amd.scenario import fdm as F  # noqa: E402

OUT = Path(__file__).resolve().parent / "fdm.json"
# name, spec, envs, input seed, steps
CASES = [
    ("fdm_small", F.FdmSpec(rows=120, cols=90, rooms=7, margin=6, seed=3), 3, 11, 10),
    ("fdm_train1_size", F.FdmSpec(), 2, 12, 3),
]


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, np.float64).tobytes()).hexdigest()


def run_case(name, spec, G, seed, steps, tmp: Path) -> dict:
    import pyoracle as po

    plan = F.make_plan(spec)
    data = F.fdm_writer(plan).tobytes()
    path = tmp / f"{name}.sbb"
    path.write_bytes(data)
    ref = po.Fdm("ref", path, G)
    probe = plan.solved[np.linspace(0, plan.n - 1, 4).astype(np.int64)]   # quantiles of the solved cells
    rec = {"spec": spec.__dict__, "envs": G, "seed": seed, "steps": steps,
           "blob_sha256": hashlib.sha256(data).hexdigest(), "probe_cells": probe.tolist(),
           "S_sha256": digest(ref.sensed_response()), "T": [], "M": [], "T_probe": []}
    for s in range(steps):
        ref.step(F.step_inputs(plan, G, seed, s))
        T, M = ref.state()
        rec["T"].append([digest(T[g]) for g in range(G)])
        rec["M"].append([digest(M[g]) for g in range(G)])
        rec["T_probe"].append(T[:, probe].tolist())
    ref.close()
    return rec


def main() -> None:
    import pyoracle as po

    if not po.ref_available():
        raise SystemExit("oracle/_ref is not built (needs /root/reference)")
    out = {}
    with tempfile.TemporaryDirectory() as td:
        for name, spec, G, seed, steps in CASES:
            out[name] = run_case(name, spec, G, seed, steps, Path(td))
            print(name, "ok", flush=True)
    OUT.write_text(json.dumps(out, indent=1))


if __name__ == "__main__":
    main()
