"""Shared-policy rollout step on the GPU, through the C ABI.

  - the MFMA MLP's head outputs against a float64 CPU evaluation of the same
    weights on the same observations (fp32 products with K up to 1024:
    within 2e-5 of the largest head value);
  - the Beta sampler against the law it draws from (mean, variance,
    Kolmogorov-Smirnov against scipy's Beta CDF), in (0, 1), deterministic;
  - the action rows: continuous heads in [-1, 1], discrete heads in {0, 1},
    zero past each env's action counts, a function of (seed, step) only;
  - a rollout where the policy's actions drive the env: the oracle stepped
    with the same action rows stays within the physics tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

import pyoracle as po

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from neurips2026_smart_building_challenge_amd import env as E  # noqa: E402


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.synchronize()


def reference_heads(obs: np.ndarray, w: dict) -> np.ndarray:
    W = {k: v.detach().cpu().double().numpy() for k, v in w.items()}
    h1 = np.tanh(obs.astype(np.float64) @ W["w1"] + W["b1"])
    h2 = np.tanh(h1 @ W["w2"] + W["b2"])
    return h2 @ W["w3"] + W["b3"]


def test_gpu_policy_heads_and_actions(mixed_dir):
    print("policy: 60 mixed envs, heads vs float64 reference", flush=True)
    vec = E.VecEnv(60, blob_dir=str(mixed_dir), groups=30, max_steps=40)
    w = E.policy_weights(123)
    vec.policy_bind(w)
    vec.reset()
    for s in range(3):                       # a few steps so observations are not reset values only
        vec.gen_actions(5, s)
        vec.step()
    vec.policy_act(7, 0)
    torch.cuda.synchronize()
    obs = vec.obs.cpu().numpy()
    y = vec.policy_heads()
    yr = reference_heads(obs, w)
    err = np.max(np.abs(y - yr)) / max(1.0, np.max(np.abs(yr)))
    assert err <= 2e-5, err
    act = vec.actions.cpu().numpy()
    for i in range(vec.n):
        nc, nd = vec.envs[i].n_cont, vec.envs[i].n_disc
        cont, disc = act[i, :256], act[i, 256:272]
        assert np.all(np.abs(cont[:nc]) < 1.0) and np.all(cont[nc:] == 0.0)
        assert set(np.unique(disc[:nd])) <= {0.0, 1.0} and np.all(disc[nd:] == 0.0)
    first = act.copy()
    vec.policy_act(7, 0)
    torch.cuda.synchronize()
    assert np.array_equal(vec.actions.cpu().numpy(), first), "actions are a function of (seed, step)"
    vec.policy_act(7, 1)
    torch.cuda.synchronize()
    assert not np.array_equal(vec.actions.cpu().numpy()[:, :64], first[:, :64])
    vec.close()


@pytest.mark.parametrize("a,b", [(1.0, 1.0), (2.0, 2.0), (1.3, 5.0), (8.0, 1.5), (30.0, 30.0),
                                 (0.3, 0.5), (0.6, 2.5), (4.0, 0.45), (150.0, 300.0), (400.0, 90.0), (700.0, 650.0)])
def test_gpu_beta_sampler_law(a, b):
    """Shapes below 1 (boosted draws) and in the hundreds (where 1 - t + log t would
    cancel) included."""
    from scipy import stats

    n = 200_000
    alpha = torch.full((n,), a, dtype=torch.float32, device="cuda")
    beta = torch.full((n,), b, dtype=torch.float32, device="cuda")
    x = E.beta_sample(alpha, beta, seed=11)
    x2 = E.beta_sample(alpha, beta, seed=11)
    torch.cuda.synchronize()
    assert torch.equal(x, x2)
    x = x.cpu().double().numpy()
    if min(a, b) >= 1.0:
        assert np.all(x > 0.0) and np.all(x < 1.0)
    else:
        assert np.all(x >= 0.0) and np.all(x <= 1.0)
    mean = a / (a + b)
    var = a * b / ((a + b) ** 2 * (a + b + 1))
    assert abs(x.mean() - mean) < 5 * np.sqrt(var / n)
    assert abs(x.var() - var) < 0.02 * var + 1e-4
    assert stats.kstest(x, stats.beta(a, b).cdf).pvalue > 1e-4


def test_gpu_policy_rollout_parity(mixed_dir):
    """30 envs (one per scenario) driven by the policy for 70 steps (one auto-reset):
    the oracle, stepped with the same action rows, agrees to the physics tolerance."""
    print("policy rollout: 30 envs x 70 steps vs oracle", flush=True)
    vec = E.VecEnv(30, blob_dir=str(mixed_dir), groups=30, max_steps=50)
    vec.policy_bind(E.policy_weights(99))
    twins = []
    for i in range(vec.n):
        path, start, seed = vec.meta(i)
        twins.append(po.CpuEnv("oracle", path, seed, start=start, max_steps=50))
    vec.reset()
    for t in twins:
        t.reset()
    for s in range(70):
        vec.policy_act(3, s)
        torch.cuda.synchronize()
        rows = vec.actions.cpu().numpy()
        vec.step()
        torch.cuda.synchronize()
        rew = vec.rewards.cpu().numpy()
        for i, t in enumerate(twins):
            _, r, term, _ = t.step(rows[i])
            assert abs(float(rew[i]) - r) <= 2 * np.spacing(np.float32(abs(r))) + 1e-12, (s, i)
            if s % 10 == 9:
                g, c = vec.state(i), t.state()
                g = g[:len(c)]
                fin = ~np.isnan(g)
                rel = np.abs(g[fin] - c[fin]) / np.maximum(np.abs(c[fin]), 1e-6)
                assert rel.max() <= 1e-9, (s, i, rel.max())
    vec.close()


def _softplus32(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.float32)
    return np.where(x > 20.0, x, np.log1p(np.exp(x)).astype(np.float32)).astype(np.float32)


def _beta_ref(u, v, x, floor=1.0):
    """float64 log-density and entropy (scipy) at the float32 shapes."""
    from scipy import stats

    a = (_softplus32(u) + np.float32(floor)).astype(np.float64)
    b = (_softplus32(v) + np.float32(floor)).astype(np.float64)
    xc = np.clip(x.astype(np.float64), 2.0**-24, 1.0 - 2.0**-24)
    return stats.beta.logpdf(xc, a, b), stats.beta.entropy(a, b)


def test_gpu_beta_eval_matches_scipy(mixed_dir):
    """sbx_beta_eval against scipy.stats.beta: per-env sums of log-densities and
    entropies over the used heads, and the per-head derivatives in u and v
    against central differences of scipy's log-density and entropy."""
    print("beta eval: 30 envs vs scipy", flush=True)
    vec = E.VecEnv(30, blob_dir=str(mixed_dir), groups=30)
    vec.policy_bind(E.policy_weights(3))
    rng = np.random.default_rng(11)
    y = rng.normal(0.0, 2.0, (vec.n, E.POLICY_HEADS)).astype(np.float32)
    y[:, :8] = [-30.0, -5.0, 0.0, 5.0, 19.9, 20.1, 30.0, 1e-3]   # both softplus branches, flat and peaked heads
    x = rng.uniform(0.0, 1.0, (vec.n, E.SB_ACT)).astype(np.float32)
    x[:, :3] = [0.0, 1.0, 0.5]                                   # the clamp at both ends
    yt, xt = torch.from_numpy(y).cuda(), torch.from_numpy(x).cuda()
    logp, ent, g = vec.beta_eval(yt, xt)
    torch.cuda.synchronize()
    logp, ent, g = logp.cpu().numpy(), ent.cpu().numpy(), g.cpu().numpy()
    for i in range(vec.n):
        nc, nd = vec.envs[i].n_cont, vec.envs[i].n_disc
        heads = list(range(nc)) + [256 + d for d in range(nd)]
        u = np.array([y[i, h] if h < 256 else y[i, 512 + h - 256] for h in heads], np.float32)
        v = np.array([y[i, 256 + h] if h < 256 else y[i, 528 + h - 256] for h in heads], np.float32)
        lp, en = _beta_ref(u, v, x[i, heads])
        assert abs(logp[i] - lp.sum()) <= 2e-5 * max(1.0, np.abs(lp).sum()), (i, logp[i], lp.sum())
        assert abs(ent[i] - en.sum()) <= 2e-5 * max(1.0, np.abs(en).sum()), (i, ent[i], en.sum())
        unused = np.setdiff1d(np.arange(E.SB_ACT), heads)
        assert np.all(g[i][:, unused] == 0.0)
        if i < 3:
            hh = 1e-3
            for which, k_lp, k_en in ((0, 0, 2), (1, 1, 3)):
                up, um = (u + hh, u - hh) if which == 0 else (u, u)
                vp, vm = (v, v) if which == 0 else (v + hh, v - hh)
                lpp, enp = _beta_ref(up.astype(np.float64), vp.astype(np.float64), x[i, heads])
                lpm, enm = _beta_ref(um.astype(np.float64), vm.astype(np.float64), x[i, heads])
                for got, want in ((g[i][k_lp, heads], (lpp - lpm) / (2 * hh)), (g[i][k_en, heads], (enp - enm) / (2 * hh))):
                    assert np.all(np.abs(got - want) <= 2e-3 * np.maximum(1.0, np.abs(want))), (i, which)
    vec.close()


def test_gpu_policy_act_logp_consistent(mixed_dir):
    """sbx_policy_act_logp draws exactly what sbx_policy_act draws (same action
    rows), records the draws behind them (continuous 2x - 1, discrete x > 0.5)
    and their log-probability and entropy, which equal sbx_beta_eval of the
    same heads and draws."""
    print("policy act with log-probabilities: 60 envs", flush=True)
    vec = E.VecEnv(60, blob_dir=str(mixed_dir), groups=30, max_steps=40)
    vec.policy_bind(E.policy_weights(5))
    vec.reset()
    vec.policy_act(9, 4)
    a_plain = vec.actions.clone()
    draws, logp, ent = vec.policy_act_logp(9, 4)
    torch.cuda.synchronize()
    assert torch.equal(vec.actions, a_plain)
    y = torch.from_numpy(vec.policy_heads()).cuda()
    lp2, en2, _ = vec.beta_eval(y, draws, grad=False)
    torch.cuda.synchronize()
    assert torch.allclose(logp, lp2, rtol=1e-6, atol=1e-5) and torch.allclose(ent, en2, rtol=1e-6, atol=1e-5)
    d, a = draws.cpu().numpy(), vec.actions.cpu().numpy()
    for i in range(vec.n):
        nc, nd = vec.envs[i].n_cont, vec.envs[i].n_disc
        assert np.all((d[i, :nc] > 0.0) & (d[i, :nc] < 1.0))
        assert np.array_equal(a[i, :nc], (np.float32(2.0) * d[i, :nc] - np.float32(1.0)).astype(np.float32))
        assert np.array_equal(a[i, 256:256 + nd], (d[i, 256:256 + nd] > 0.5).astype(np.float32))
        assert np.all(d[i, nc:256] == 0.0) and np.all(d[i, 256 + nd:] == 0.0)
    vec.close()


def _heads_of(vec, i):
    nc, nd = vec.envs[i].n_cont, vec.envs[i].n_disc
    heads = list(range(nc)) + [256 + d for d in range(nd)]
    cu = np.array([h if h < 256 else 512 + h - 256 for h in heads])
    cv = np.array([256 + h if h < 256 else 528 + h - 256 for h in heads])
    return np.array(heads), cu, cv


def _shapes(y, floor):
    return (_softplus32(y) + np.float32(floor)).astype(np.float64)


def _ppo_ref(yn, yo, x, lp_old, adv, floor, clip, ent_coef, per_dim):
    """float64 restatement from scipy.stats.beta (log-density, entropy), the KL
    closed form (pinned against quadrature in tests/test_policy_math.py) and the
    clipped surrogate of Schulman et al. 2017: (logp, H, KL, r, pg, lr, loss)."""
    from scipy import stats

    from test_policy_math import beta_kl

    an, bn = _shapes(yn[0], floor), _shapes(yn[1], floor)
    ao, bo = _shapes(yo[0], floor), _shapes(yo[1], floor)
    xc = np.clip(x.astype(np.float64), 2.0**-24, 1.0 - 2.0**-24)
    lp = stats.beta.logpdf(xc, an, bn).sum()
    en = stats.beta.entropy(an, bn).sum()
    kl = beta_kl(ao, bo, an, bn).sum()
    D = len(x)
    lr = (lp - lp_old) / (D if per_dim else 1)
    lr = min(20.0, max(-20.0, lr))
    r = np.exp(lr)
    pg = (D if per_dim else 1) * max(-adv * r, -adv * min(1 + clip, max(1 - clip, r)))
    return lp, en, kl, r, pg, lr, pg - ent_coef * en


@pytest.mark.parametrize("floor,per_dim", [(1.0, True), (1.0, False), (0.25, True)])
def test_gpu_ppo_beta_matches_reference(mixed_dir, floor, per_dim):
    """sbx_ppo_beta against a float64 evaluation: per-env log-probability, entropy,
    KL(old || new), ratio, clipped surrogate and log-ratio; the per-head gradients of
    pg - ent_coef H in u and v against central differences of that evaluation (on
    heads whose ratio is inside and outside the clip range). floor 0.25 exercises
    shapes below 1."""
    print(f"ppo beta: floor {floor}, ratio_per_dim {per_dim}", flush=True)
    vec = E.VecEnv(30, blob_dir=str(mixed_dir), groups=30)
    rng = np.random.default_rng(5)
    yn = rng.normal(0.0, 1.5, (vec.n, E.POLICY_HEADS)).astype(np.float32)
    yo = (yn + rng.normal(0.0, 0.05, yn.shape)).astype(np.float32)
    x = rng.uniform(0.02, 0.98, (vec.n, E.SB_ACT)).astype(np.float32)
    clip, ent_coef = 0.2, 0.01
    lp_old = np.zeros(vec.n, np.float32)
    adv = rng.normal(0.0, 1.0, vec.n).astype(np.float32)
    refs = []
    for i in range(vec.n):
        heads, cu, cv = _heads_of(vec, i)
        ref0 = _ppo_ref((yn[i, cu], yn[i, cv]), (yo[i, cu], yo[i, cv]), x[i, heads], 0.0, adv[i], floor, clip,
                        ent_coef, per_dim)
        # stored log-probabilities that put half the envs' ratios outside the clip range
        shift = (0.5 if i % 2 else 0.02) * (len(heads) if per_dim else 1)
        lp_old[i] = np.float32(ref0[0] + (shift if i % 4 < 2 else -shift))
        refs.append((heads, cu, cv))
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    out, g = vec.ppo_beta(T(yn), T(yo), T(x), T(lp_old), T(adv), clip, ent_coef, per_dim, floor)
    torch.cuda.synchronize()
    out, g = out.cpu().numpy(), g.cpu().numpy()
    clipped = 0
    for i in range(vec.n):
        heads, cu, cv = refs[i]
        ref = _ppo_ref((yn[i, cu], yn[i, cv]), (yo[i, cu], yo[i, cv]), x[i, heads], float(lp_old[i]), float(adv[i]),
                       floor, clip, ent_coef, per_dim)
        for k in range(6):
            tol = 2e-5 * max(1.0, abs(ref[k])) if k != 3 else 1e-4 * ref[3]
            assert abs(out[i, k] - ref[k]) <= tol, (i, k, out[i, k], ref[k])
        clipped += abs(ref[3] - 1.0) > clip
        unused = np.setdiff1d(np.arange(E.SB_ACT), heads)
        assert np.all(g[i][:, unused] == 0.0)
        if i < 6:
            hh = 1e-3
            for which, cols in ((0, cu), (1, cv)):
                for j in range(0, len(heads), 7):
                    yp, ym = yn[i].astype(np.float64), yn[i].astype(np.float64)
                    yp, ym = yp.copy(), ym.copy()
                    yp[cols[j]] += hh
                    ym[cols[j]] -= hh
                    fp = _ppo_ref((yp[cu], yp[cv]), (yo[i, cu], yo[i, cv]), x[i, heads], float(lp_old[i]),
                                  float(adv[i]), floor, clip, ent_coef, per_dim)[6]
                    fm = _ppo_ref((ym[cu], ym[cv]), (yo[i, cu], yo[i, cv]), x[i, heads], float(lp_old[i]),
                                  float(adv[i]), floor, clip, ent_coef, per_dim)[6]
                    want = (fp - fm) / (2 * hh)
                    assert abs(g[i, which, heads[j]] - want) <= 2e-3 * max(1.0, abs(want)), (i, which, j)
    assert 0 < clipped < vec.n
    vec.close()


def test_gpu_beta_eval_floor_below_one(mixed_dir):
    """sbx_beta_eval with a shape floor of 0.25 (shapes below 1) against scipy."""
    print("beta eval, floor 0.25", flush=True)
    vec = E.VecEnv(30, blob_dir=str(mixed_dir), groups=30)
    vec.policy_bind(E.policy_weights(3), beta_floor=0.25)
    rng = np.random.default_rng(12)
    y = rng.normal(-1.0, 2.0, (vec.n, E.POLICY_HEADS)).astype(np.float32)
    x = rng.uniform(0.0, 1.0, (vec.n, E.SB_ACT)).astype(np.float32)
    logp, ent, _ = vec.beta_eval(torch.from_numpy(y).cuda(), torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    logp, ent = logp.cpu().numpy(), ent.cpu().numpy()
    for i in range(vec.n):
        heads, cu, cv = _heads_of(vec, i)
        lp, en = _beta_ref(y[i, cu], y[i, cv], x[i, heads], floor=0.25)
        assert abs(logp[i] - lp.sum()) <= 2e-5 * max(1.0, np.abs(lp).sum()), (i, logp[i], lp.sum())
        assert abs(ent[i] - en.sum()) <= 2e-5 * max(1.0, np.abs(en).sum()), (i, ent[i], en.sum())
    # the policy with that floor draws inside [0, 1] and writes legal action rows
    vec.reset()
    vec.policy_act(3, 0)
    torch.cuda.synchronize()
    act = vec.actions.cpu().numpy()
    assert np.all(np.abs(act[:, :256]) <= 1.0) and set(np.unique(act[:, 256:])) <= {0.0, 1.0}
    vec.close()
