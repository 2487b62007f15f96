"""Shared fixtures. GPU tests carry @pytest.mark.gpu; everything else runs on CPU."""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP env step)")
    config.addinivalue_line("markers", "slow: longer CPU checks")


@pytest.fixture(scope="session")
def golden_index() -> dict:
    return json.loads((GOLDEN / "golden.json").read_text())


def golden_blob(layout, climate, out_dir: Path, conv=None) -> tuple[Path, str]:
    """Regenerates the blob of a golden case (conv: (p, distance, seed) or None);
    returns (path, sha256)."""
    from neurips2026_smart_building_challenge_amd.scenario import generate as G

    spec = G.LayoutSpec(*layout)
    clim = G.ClimateSpec(climate[0], climate[1], seed=climate[2])
    cv = None if conv is None else G.ConvSpec(*conv)
    p = out_dir / f"{spec.name}__{clim.name}{'' if cv is None else '__' + cv.tag}.sbb"
    data = G.scenario_writer(spec, clim, 2 * G.EPISODE_STEPS, 17321, cv).tobytes()
    p.write_bytes(data)
    return p, hashlib.sha256(data).hexdigest()


@pytest.fixture(scope="session")
def mixed_dir(tmp_path_factory) -> Path:
    """The 30 scenarios of the 960-env config (6 layouts x 5 climates)."""
    from neurips2026_smart_building_challenge_amd.scenario import generate as G

    d = tmp_path_factory.mktemp("mixed")
    G.write_config(1, d)
    return d


@pytest.fixture(scope="session")
def cfg0_dir(tmp_path_factory) -> Path:
    from neurips2026_smart_building_challenge_amd.scenario import generate as G

    d = tmp_path_factory.mktemp("cfg0")
    G.write_config(0, d)
    return d


def conv_scenarios(out_dir: Path, p: float, distance: int, seed: int) -> Path:
    """The 6 layouts under one climate with stochastic convection on."""
    from neurips2026_smart_building_challenge_amd.scenario import generate as G

    scen = [(G.LayoutSpec(z, a), G.ClimateSpec(12.0, 8.0, seed=502)) for z, a in G.LAYOUTS]
    G.write_scenarios(scen, out_dir, conv=G.ConvSpec(p, distance, seed))
    return out_dir


@pytest.fixture(scope="session")
def conv_dir(tmp_path_factory) -> Path:
    return conv_scenarios(tmp_path_factory.mktemp("conv"), 0.08, 2, 4242)
