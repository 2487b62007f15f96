"""The allocation-free policy entry point (sbx_policy_act_noalloc) against the
one it varies (sbx_policy_bind + sbx_policy_act), through the C ABI: the same
action rows bit for bit on two calls in a row, the second on a smaller vec
(the shared device scratch then holds the first call's larger contents), and
the size limit rejected with a message."""
from __future__ import annotations

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from neurips2026_smart_building_challenge_amd import env as E  # noqa: E402


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.synchronize()


def _stepped(mixed_dir, n, seed):
    vec = E.VecEnv(n, blob_dir=str(mixed_dir), groups=30, max_steps=40)
    vec.reset()
    for s in range(3):
        vec.gen_actions(seed, s)
        vec.step()
    torch.cuda.synchronize()
    return vec


def test_gpu_policy_noalloc_matches_bound(mixed_dir):
    w = E.policy_weights(321)
    for n, step in ((960, 11), (100, 12)):
        print(f"no-alloc policy: {n} envs, step {step}", flush=True)
        sys.stdout.flush()
        a = _stepped(mixed_dir, n, 5)
        b = _stepped(mixed_dir, n, 5)
        assert torch.equal(a.obs, b.obs)
        a.policy_bind(w)
        a.policy_act(77, step)
        b.actions.fill_(9.0)
        b.policy_act_noalloc(w, 77, step)
        torch.cuda.synchronize()
        assert torch.equal(a.actions, b.actions), n
        act = b.actions.cpu().numpy()
        assert np.all(np.abs(act) <= 1.0)
        a.close()
        b.close()


def test_gpu_policy_noalloc_rejects_oversize(tmp_path):
    from neurips2026_smart_building_challenge_amd.scenario import generate as G

    G.write_config(0, tmp_path)
    vec = E.VecEnv(4097, blob_dir=str(tmp_path))    # SBX_NOALLOC_MAX_ENVS + 1
    with pytest.raises(RuntimeError, match="at most 4096"):
        vec.policy_act_noalloc(E.policy_weights(1), 1, 0)
    vec.close()
