"""GPU: the engine's sampling kernel against the reference sampling rule
(src/infer.py:658-685), through `pulsar_sample_rows`.

* The penalised argmax is exact (lowest index on ties), in fp32 and bf16 rounding.
* Every draw lies in the top-p set: the tokens whose probability mass strictly above them
  is at most top_p, evaluated in fp64 on the scores rounded as the kernel's dtype rounds
  them (ties kept or dropped together; a token within 1e-5 of the cut may go either way).
* The draws of 4096 independent streams over one distribution match the renormalised
  top-p probabilities (chi-square, significance 1e-6).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

V = 32768


def _scores(row: np.ndarray, seen: set, extra: int, rp: float, temperature: float, bf16: bool):
    l = torch.tensor(row, dtype=torch.float32)
    rnd = (lambda t: t.to(torch.bfloat16).float()) if bf16 else (lambda t: t)  # noqa: E731
    ids = set(seen) | ({extra} if extra >= 0 else set())
    for t in ids:
        v = l[t]
        l[t] = rnd(v / rp if v > 0 else v * rp)
    arg = int(torch.argmax(l))
    return arg, rnd(l / temperature).double()


def _top_p(s: torch.Tensor, top_p: float):
    p = torch.softmax(s, dim=0)
    order = torch.argsort(s, descending=True, stable=True)
    sp, ss = p[order], s[order]
    # mass strictly above each token: cumulative mass before the first token of its tie group
    cum = torch.cumsum(sp, 0) - sp
    first = torch.ones_like(ss, dtype=torch.bool)
    first[1:] = ss[1:] != ss[:-1]
    grp = torch.cumsum(first.long(), 0) - 1
    above_sorted = cum[first][grp]
    above = torch.empty_like(above_sorted)
    above[order] = above_sorted
    kept = above <= top_p
    ambiguous = (above - top_p).abs() <= 1e-5
    return p, kept, ambiguous


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_argmax_exact_and_draws_inside_top_p(dtype):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pulsar_engine.engine import sample_rows

    rng = np.random.default_rng(3)
    n, n_seq = 64, 8
    rows = rng.normal(0, 2.5, size=(n, V)).astype(np.float32)
    rows[::4] = np.round(rows[::4] * 4) / 4          # many exact ties
    rows[1::8, 77] = 40.0                              # one dominant token
    rows[2::8, :] = 0.0                                # a flat row: every token tied
    rows[3::8, 4100] = rows[3::8, 9000] = 40.0         # two tied dominant tokens
    seen = [set(rng.integers(0, V, 120).tolist()) | {77} for _ in range(n_seq)]
    row_seq = [i % n_seq for i in range(n)]
    row_extra = [int(rng.integers(0, V)) if i % 3 == 0 else -1 for i in range(n)]
    ctr = list(range(n_seq))
    T, top_p, rp = 0.8, 0.9, 1.15
    bf16 = dtype == torch.bfloat16
    am, dr = sample_rows(torch.from_numpy(rows).cuda(), seen, row_seq, row_extra, ctr, 1234, T,
                         top_p, rp, dtype=dtype)
    for i in range(n):
        arg, s = _scores(rows[i], seen[row_seq[i]], row_extra[i], rp, T, bf16)
        assert am[i] == arg, (i, am[i], arg)
        _, kept, amb = _top_p(s, top_p)
        for d in range(2):
            t = int(dr[i, d])
            assert 0 <= t < V and (bool(kept[t]) or bool(amb[t])), (i, d, t)
    greedy_am, greedy_dr = sample_rows(torch.from_numpy(rows).cuda(), seen, row_seq, row_extra,
                                       ctr, 1234, T, top_p, rp, greedy=True, dtype=dtype)
    assert (greedy_am == am).all() and (greedy_dr == am[:, None]).all()


def test_draw_frequencies_follow_top_p_distribution():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from scipy.stats import chi2

    from pulsar_engine.engine import sample_rows

    rng = np.random.default_rng(5)
    row = rng.normal(0, 1.0, size=V).astype(np.float32)
    row[rng.choice(V, 40, replace=False)] += rng.uniform(6.0, 9.0, 40).astype(np.float32)
    n = 2048
    T, top_p, rp = 0.8, 0.95, 1.0
    # one sequence (and so one counter stream) per row: 2n independent draws
    am, dr = sample_rows(torch.from_numpy(np.tile(row, (n, 1))).cuda(), [[] for _ in range(n)],
                         list(range(n)), [-1] * n, list(range(n)), 99, T, top_p, rp,
                         dtype=torch.float32)
    _, s = _scores(row, set(), -1, rp, T, False)
    p, kept, _ = _top_p(s, top_p)
    q = torch.where(kept, p, torch.zeros_like(p))
    q = (q / q.sum()).numpy()
    draws = dr.reshape(-1)
    assert kept[torch.from_numpy(draws.astype(np.int64))].all()
    counts = np.bincount(draws, minlength=V).astype(np.float64)
    expected = q * draws.size
    big = expected >= 5
    obs = np.append(counts[big], counts[~big].sum())
    exp = np.append(expected[big], expected[~big].sum())
    keep = exp > 0
    stat = float(((obs[keep] - exp[keep]) ** 2 / exp[keep]).sum())
    df = int(keep.sum()) - 1
    print(f"chi-square {stat:.1f} on {df} degrees of freedom, {int(kept.sum())} kept tokens")
    assert stat < chi2.ppf(1 - 1e-6, df)
